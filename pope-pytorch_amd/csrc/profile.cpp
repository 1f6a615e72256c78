// Opt-in per-kernel timing: when enabled, every kernel launch of the library carries a pair of
// hipEvents that its dispatch stamps with the kernel's own start and end times.
// Reading the totals waits for the recorded events, folds their elapsed times
// into per-kernel statistics and returns the event pairs to a pool.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "pope_kernels.hpp"

namespace pope {

namespace {

struct Pending {
  const char* name;
  hipEvent_t a, b;
  bool live;
};

struct Stat {
  long count = 0;
  double total_ms = 0.0, min_ms = 1e30, max_ms = 0.0;
};

std::atomic<int> g_on{0};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_pool;
std::map<std::string, Stat> g_stats;
constexpr size_t kMaxPending = 1 << 16;

}  // namespace

int prof_begin(const char* name, hipEvent_t* start, hipEvent_t* stop) {
  if (!g_on.load(std::memory_order_relaxed)) return -1;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_pending.size() >= kMaxPending) return -1;
  Pending p{name, nullptr, nullptr, true};
  if (!g_pool.empty()) {
    p.a = g_pool.back().first;
    p.b = g_pool.back().second;
    g_pool.pop_back();
  } else if (hipEventCreate(&p.a) != hipSuccess) {
    return -1;
  } else if (hipEventCreate(&p.b) != hipSuccess) {
    (void)hipEventDestroy(p.a);
    return -1;
  }
  g_pending.push_back(p);
  *start = p.a;
  *stop = p.b;
  return (int)g_pending.size() - 1;
}

void prof_cancel(int token) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (token >= 0 && (size_t)token < g_pending.size()) g_pending[token].live = false;
}

void prof_enable(int on) { g_on.store(on ? 1 : 0); }

// Waits for every pending pair, accumulates, then writes
// "name count total_ms min_ms max_ms" lines into buf.
int prof_read(char* buf, size_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = 0;
  for (const Pending& p : g_pending) {
    float ms = 0.f;
    if (!p.live) {
      g_pool.emplace_back(p.a, p.b);
      continue;
    }
    if (hipEventSynchronize(p.b) != hipSuccess || hipEventElapsedTime(&ms, p.a, p.b) != hipSuccess) {
      rc = 1;
    } else {
      Stat& st = g_stats[p.name];
      st.count += 1;
      st.total_ms += ms;
      if (ms < st.min_ms) st.min_ms = ms;
      if (ms > st.max_ms) st.max_ms = ms;
    }
    g_pool.emplace_back(p.a, p.b);
  }
  g_pending.clear();
  std::string out;
  char line[256];
  for (const auto& kv : g_stats) {
    snprintf(line, sizeof line, "%s %ld %.6f %.6f %.6f\n", kv.first.c_str(), kv.second.count, kv.second.total_ms,
             kv.second.min_ms, kv.second.max_ms);
    out += line;
  }
  if (buf && n) {
    const size_t m = out.size() < n - 1 ? out.size() : n - 1;
    out.copy(buf, m);
    buf[m] = '\0';
    if (out.size() >= n) rc = rc ? rc : 2;
  }
  return rc;
}

void prof_reset() {
  std::lock_guard<std::mutex> lk(g_mu);
  g_stats.clear();
}

}  // namespace pope
