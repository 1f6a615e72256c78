// C ABI of libpope_hip.so: host-side validation, workspace layout and dispatch.
// Declarations and the reference interfaces they replace: include/pope_abi.h.
#include "../../include/pope_abi.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "pope_kernels.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(POPE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
int round_up(int x, int m) { return (x + m - 1) / m * m; }

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// Geometry shared by the ops.
struct Geo {
  int Bt, Ht;   // phase-table batch / head extents (1 when freqs broadcasts)
  size_t table; // bytes of a (Bt, Ht, Nk, R) float2 table
};

Geo geometry(const pope_desc& d, int heads) {
  Geo g;
  g.Bt = d.f_s[0] != 0 ? d.B : 1;
  g.Ht = d.f_s[1] != 0 ? heads : 1;
  g.table = d.R > 0 ? align_up((size_t)g.Bt * g.Ht * d.Nk * d.R * sizeof(float2)) : 0;
  return g;
}

int check_strides16(const char* name, const int64_t* s) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] % 8) != 0)
      return fail(POPE_ERR_INVALID, "%s stride[%d] = %lld must be a non-negative multiple of 8 elements",
                  name, i, (long long)s[i]);
  return POPE_OK;
}

int check_strides32(const char* name, const int64_t* s) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] % 4) != 0)
      return fail(POPE_ERR_INVALID, "%s stride[%d] = %lld must be a non-negative multiple of 4 elements",
                  name, i, (long long)s[i]);
  return POPE_OK;
}

// Checks common to every op.
int check_desc(const pope_desc* d) {
  if (!d) return fail(POPE_ERR_INVALID, "descriptor is NULL");
  if (d->B < 1 || d->Hq < 1 || d->Hk < 1 || d->Nq < 1 || d->Nk < 1)
    return fail(POPE_ERR_INVALID, "B, Hq, Hk, Nq, Nk must be >= 1 (got %d, %d, %d, %d, %d)", d->B, d->Hq,
                d->Hk, d->Nq, d->Nk);
  if (d->Hq % d->Hk != 0)
    return fail(POPE_ERR_INVALID, "query heads %d must be a multiple of kv heads %d", d->Hq, d->Hk);
  if (d->D < 8 || d->D % 8 != 0)
    return fail(POPE_ERR_INVALID, "head dim %d must be a positive multiple of 8", d->D);
  if (d->R < 0 || d->R > d->D || d->R % 8 != 0)
    return fail(POPE_ERR_INVALID, "rotate dim %d must be a multiple of 8 in [0, head dim %d]", d->R, d->D);
  if (d->R > 0 && d->Nq > d->Nk)
    return fail(POPE_ERR_INVALID, "query length %d exceeds key length %d (q rows are right-aligned)", d->Nq,
                d->Nk);
  if (d->f_s[0] < 0 || d->f_s[1] < 0 || d->f_s[2] < 0 || d->bias_sh < 0)
    return fail(POPE_ERR_INVALID, "negative freqs/bias stride");
  if (d->R > 0 && d->f_s[1] != 0 && d->Hq != d->Hk)
    return fail(POPE_ERR_UNSUPPORTED, "per-head freqs need Hq == Hk");
  return POPE_OK;
}

int check_pope_ptrs(const pope_desc* d, const float* freqs, const float* bias) {
  if (d->R > 0 && (!freqs || !bias))
    return fail(POPE_ERR_INVALID, "rotate dim %d > 0 needs freqs and bias", d->R);
  return POPE_OK;
}

int check_ws(size_t need, void* ws, size_t have) {
  if (need == 0) return POPE_OK;
  if (!ws || have < need)
    return fail(POPE_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws ? have : (size_t)0);
  if ((reinterpret_cast<uintptr_t>(ws) % kAlign) != 0)
    return fail(POPE_ERR_WORKSPACE, "workspace must be %zu-byte aligned", kAlign);
  return POPE_OK;
}

// Deterministic-mode region at the end of a backward's workspace (POPE_FLAG_DETERMINISTIC):
//   dpsi (B, Hk, Nk, R) | dphi (B, Hq, Nq, R) | dbias slices            fp32
// The kernels write every phase derivative once; launch_phase_grad_reduce sums them in a fixed
// order into dfreqs / dbias.
size_t det_bytes(const pope_desc& d) {
  if (!(d.flags & POPE_FLAG_DETERMINISTIC) || d.R == 0) return 0;
  const int Hb = d.bias_sh != 0 ? d.Hk : 1;
  return align_up((size_t)d.B * d.Hk * d.Nk * d.R * sizeof(float)) +
         align_up((size_t)d.B * d.Hq * d.Nq * d.R * sizeof(float)) +
         align_up(pope::phase_grad_slices(Hb, d.R) * sizeof(float));
}

struct DetParts {
  float* kpart;
  float* qpart;
  float* slices;
};

// The region at `base`; null pointers outside deterministic mode, and for parts nothing reads
// (kpart feeds dfreqs and dbias, qpart dfreqs only).
DetParts det_parts(const pope_desc& d, char* base, const float* dfreqs, const float* dbias) {
  DetParts r{nullptr, nullptr, nullptr};
  if (!det_bytes(d) || (!dfreqs && !dbias)) return r;
  const size_t kb = align_up((size_t)d.B * d.Hk * d.Nk * d.R * sizeof(float));
  const size_t qb = align_up((size_t)d.B * d.Hq * d.Nq * d.R * sizeof(float));
  r.kpart = reinterpret_cast<float*>(base);
  r.qpart = dfreqs ? reinterpret_cast<float*>(base + kb) : nullptr;
  r.slices = reinterpret_cast<float*>(base + kb + qb);
  return r;
}

hipError_t det_reduce(const pope_desc& d, const DetParts& dp, float* dfreqs, float* dbias, bool overwrite,
                      hipStream_t s) {
  if (!dp.kpart) return hipSuccess;
  pope::PhaseGradParams g;
  std::memset(&g, 0, sizeof g);
  g.kpart = dp.kpart;
  g.qpart = dp.qpart;
  g.dfreqs = dfreqs;
  g.dbias = dbias;
  g.bslices = dp.slices;
  g.B = d.B; g.Hq = d.Hq; g.Hk = d.Hk; g.Nq = d.Nq; g.Nk = d.Nk; g.R = d.R;
  g.Bt = d.f_s[0] != 0 ? d.B : 1;
  g.Ht = d.f_s[1] != 0 ? d.Hq : 1;   // per-head tables need Hq == Hk
  g.Hb = d.bias_sh != 0 ? d.Hk : 1;
  g.overwrite = overwrite ? 1 : 0;
  g.df_s[0] = d.df_s[0]; g.df_s[1] = d.df_s[1]; g.df_s[2] = d.df_s[2];
  g.bias_sh = d.bias_sh;
  return pope::launch_phase_grad_reduce(g, s);
}

// Flash forward / backward workspace (the same layout for both, so the backward can reuse the
// forward's preparation), each piece 256-byte aligned:
//   cos/sin(F) (Bt, Ht, Nk, R) float2 | cos/sin(bias) (Hb, R) float2
//   | K_hat (B, Hk, NkP, EP) | Q_hat (B, Hq, NqP, EP)      16-bit elements
//   | key visibility words (B, NW) u64 | last visible key + 1 (B) int32
//   | -lse * log2 e, -delta (B, Hq, NqP) fp32 each           backward only
// with EP = round_up(D + R, 32), DV = round_up(D, 32), NqP / NkP = round_up(N, 256) (the backward's
// jobs cover 256 rows), NW = NkP / 64.  Wide heads (D > 128, flash_wide.hip): EP =
// round_up(D + R, 128), DV = 256, and the backward's workspace adds the raw expanded-row
// gradients, fp32 (B, Hk, NkP, EP) and (B, Hq, NqP, EP), before the deterministic-mode region.
void copy3(int64_t* dst, const int64_t* src);

struct FlashLayout {
  int EP, DV, NqP, NkP, NW, Bt, Ht, Hb;
  bool wide;
  size_t table, btab, kh, qh, mwords, kend, ld, total;
  size_t wk, wq, wide_bytes;   // backward only, offsets past `total`
};

constexpr int kFlashMaxD = 128;       // head dims of the register-tiled kernels
constexpr int kFlashWideMaxD = 256;   // head dims of the wide kernels

FlashLayout flash_layout(const pope_desc& d) {
  FlashLayout L;
  L.wide = d.D > kFlashMaxD;
  L.EP = L.wide ? round_up(d.D + d.R, 128) : round_up(d.D + d.R, 32);
  L.DV = L.wide ? 256 : round_up(d.D, 32);
  L.NqP = round_up(d.Nq, 256);
  L.NkP = round_up(d.Nk, 256);
  L.NW = L.NkP / 64;
  L.Bt = d.f_s[0] != 0 ? d.B : 1;
  L.Ht = d.f_s[1] != 0 ? d.Hq : 1;
  L.Hb = d.bias_sh != 0 ? d.Hk : 1;
  size_t off = 0;
  L.table = off;  off += d.R > 0 ? align_up((size_t)L.Bt * L.Ht * d.Nk * d.R * sizeof(float2)) : 0;
  L.btab = off;   off += d.R > 0 ? align_up((size_t)L.Hb * d.R * sizeof(float2)) : 0;
  L.kh = off;     off += align_up((size_t)d.B * d.Hk * L.NkP * L.EP * 2);
  L.qh = off;     off += align_up((size_t)d.B * d.Hq * L.NqP * L.EP * 2);
  L.mwords = off; off += align_up((size_t)d.B * L.NW * sizeof(uint64_t));
  L.kend = off;   off += align_up((size_t)d.B * sizeof(int32_t));
  L.ld = off;     off += align_up((size_t)d.B * d.Hq * L.NqP * sizeof(float2));
  L.total = off;
  L.wk = off;
  L.wq = L.wk + (L.wide ? align_up((size_t)d.B * d.Hk * L.NkP * L.EP * sizeof(float)) : 0);
  L.wide_bytes = L.wide ? L.wq - L.wk + align_up((size_t)d.B * d.Hq * L.NqP * L.EP * sizeof(float)) : 0;
  return L;
}

// The backward's workspace extends the forward's by the wide path's raw gradients and the
// deterministic-mode region.
size_t flash_ws(const pope_desc& d, int op) {
  const FlashLayout L = flash_layout(d);
  return L.total + (op == POPE_OP_FLASH_BWD ? L.wide_bytes + det_bytes(d) : 0);
}

// The flash kernels address the rows of v and do inside one (batch, head) with 32-bit element
// offsets, up to one tile past the padded length.
int check_row_span(const char* name, int rows_padded, int64_t row_stride) {
  const int64_t span = ((int64_t)rows_padded + 256) * row_stride;
  if (span >= ((int64_t)1 << 31))
    return fail(POPE_ERR_UNSUPPORTED, "%s rows span %lld elements per (batch, head); the kernels index them "
                "with 32-bit offsets", name, (long long)span);
  return POPE_OK;
}

// Launches the shared preparation of the flash forward and backward into the workspace.
hipError_t flash_prepare(const pope_desc& d, const FlashLayout& L, const void* q, const void* k,
                         const float* freqs, const float* bias, const uint8_t* mask, char* ws, hipStream_t s) {
  pope::FlashPrep p;
  std::memset(&p, 0, sizeof p);
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.freqs = d.R > 0 ? freqs : nullptr;
  p.bias = d.R > 0 ? bias : nullptr;
  p.mask = mask;
  p.table = reinterpret_cast<float2*>(ws + L.table);
  p.btab = reinterpret_cast<float2*>(ws + L.btab);
  p.qh = reinterpret_cast<uint16_t*>(ws + L.qh);
  p.kh = reinterpret_cast<uint16_t*>(ws + L.kh);
  p.mwords = reinterpret_cast<uint64_t*>(ws + L.mwords);
  p.kend = reinterpret_cast<int*>(ws + L.kend);
  p.B = d.B; p.Hq = d.Hq; p.Hk = d.Hk; p.Nq = d.Nq; p.Nk = d.Nk; p.D = d.D; p.R = d.R;
  p.EP = L.EP; p.NqP = L.NqP; p.NkP = L.NkP; p.NW = L.NW;
  p.Bt = L.Bt; p.Ht = L.Ht; p.Hb = L.Hb;
  p.has_mask = mask != nullptr;
  p.qscale = d.softmax_scale * 1.4426950408889634f;
  copy3(p.q_s, d.q_s);
  copy3(p.k_s, d.k_s);
  copy3(p.f_s, d.f_s);
  p.bias_sh = d.bias_sh;
  p.mask_sb = d.mask_sb;
  p.t_sb = L.Bt > 1 ? (int64_t)L.Ht * d.Nk * d.R : 0;
  p.t_sh = L.Ht > 1 ? (int64_t)d.Nk * d.R : 0;
  return pope::launch_flash_prep(p, d.dtype, s);
}

// Similarity workspace: [key table with bias (Bt, Hk) | query table without bias (Bt, Hqt)
//                        | U (B, Hq, Nq, EP) | W (B, Hk, Nk, EP)]  (the last three for the backward).
size_t sim_table_k(const pope_desc& d) {
  const int Bt = d.f_s[0] != 0 ? d.B : 1;
  return d.R > 0 ? align_up((size_t)Bt * d.Hk * d.Nk * d.R * sizeof(float2)) : 0;
}
size_t sim_table_q(const pope_desc& d) {
  const int Bt = d.f_s[0] != 0 ? d.B : 1;
  const int Hqt = d.f_s[1] != 0 ? d.Hq : 1;
  return d.R > 0 ? align_up((size_t)Bt * Hqt * d.Nk * d.R * sizeof(float2)) : 0;
}
// Similarity workspace: [key table | query table | (backward) U | W | (split) Q_hat hi | lo |
// K_hat hi | lo planes, rows padded to 128].
size_t sim_ws(const pope_desc& d, int op) {
  const int EP = round_up(d.D + d.R, 32);
  size_t n = sim_table_k(d) + sim_table_q(d);
  if (op == POPE_OP_SIM_BWD) {
    n += align_up((size_t)d.B * d.Hq * d.Nq * EP * sizeof(float));
    n += align_up((size_t)d.B * d.Hk * d.Nk * EP * sizeof(float));
  }
  if (d.flags & POPE_FLAG_SPLIT_BF16) {
    n += 2 * align_up((size_t)d.B * d.Hq * round_up(d.Nq, 128) * EP * sizeof(uint16_t));
    n += 2 * align_up((size_t)d.B * d.Hk * round_up(d.Nk, 128) * EP * sizeof(uint16_t));
    if (op == POPE_OP_SIM_BWD) {   // second partial sums of U and W
      n += align_up((size_t)d.B * d.Hq * d.Nq * EP * sizeof(float));
      n += align_up((size_t)d.B * d.Hk * d.Nk * EP * sizeof(float));
    }
  }
  if (op == POPE_OP_SIM_BWD) n += det_bytes(d);   // last: its offset is sim_ws - det_bytes
  return n;
}

// The split planes at the end of the similarity workspace.
pope::SimSplit sim_split_planes(const pope_desc& d, char* ws, int op) {
  const int EP = round_up(d.D + d.R, 32);
  pope::SimSplit sp;
  sp.NqP = round_up(d.Nq, 128);
  sp.NkP = round_up(d.Nk, 128);
  size_t off = sim_table_k(d) + sim_table_q(d);
  if (op == POPE_OP_SIM_BWD)
    off += align_up((size_t)d.B * d.Hq * d.Nq * EP * sizeof(float)) + align_up((size_t)d.B * d.Hk * d.Nk * EP * sizeof(float));
  const size_t qb = align_up((size_t)d.B * d.Hq * sp.NqP * EP * sizeof(uint16_t));
  const size_t kb = align_up((size_t)d.B * d.Hk * sp.NkP * EP * sizeof(uint16_t));
  sp.qh = reinterpret_cast<uint16_t*>(ws + off);
  sp.ql = reinterpret_cast<uint16_t*>(ws + off + qb);
  sp.kh = reinterpret_cast<uint16_t*>(ws + off + 2 * qb);
  sp.kl = reinterpret_cast<uint16_t*>(ws + off + 2 * qb + kb);
  sp.U2 = sp.W2 = nullptr;
  if (op == POPE_OP_SIM_BWD) {
    const size_t o2 = off + 2 * qb + 2 * kb;
    sp.U2 = reinterpret_cast<float*>(ws + o2);
    sp.W2 = reinterpret_cast<float*>(ws + o2 + align_up((size_t)d.B * d.Hq * d.Nq * EP * sizeof(float)));
  }
  return sp;
}

// Decode workspace: [fp16 cos/sin table | partial O (rows, splits, D) | partial (m, l)
// (rows, splits, 2) | query weights (rows, D) float2], one split per pope::decode_split_keys()
// keys.
int decode_splits(const pope_desc& d) {
  const int per = pope::decode_split_keys(d.D);
  return (d.Nk + per - 1) / per;
}

size_t decode_ws(const pope_desc& d) {
  const int splits = decode_splits(d);
  const size_t rows = (size_t)d.B * d.Hq * d.Nq;
  return align_up(rows * splits * d.D * sizeof(float)) + align_up(rows * splits * 2 * sizeof(float));
}

hipError_t build_table(const pope_desc& d, const float* freqs, const float* bias, int Bt, int Ht,
                       float2* out, hipStream_t s, uint32_t* out16 = nullptr) {
  pope::TableParams t;
  t.out16 = out16;
  t.freqs = freqs;
  t.f_sb = d.f_s[0];
  t.f_sh = d.f_s[1];
  t.f_sn = d.f_s[2];
  t.bias = bias;
  t.bias_sh = d.bias_sh;
  t.Bt = Bt;
  t.Ht = Ht;
  t.rows = d.Nk;
  t.R = d.R;
  t.out = out;
  return pope::launch_phase_table(t, s);
}

void copy3(int64_t* dst, const int64_t* src) {
  dst[0] = src[0];
  dst[1] = src[1];
  dst[2] = src[2];
}

int check_flash_common(const pope_desc* d, const void* q, const void* k, const void* v, const float* freqs,
                       const float* bias, const uint8_t* mask, const void* o, const float* lse) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (d->dtype != POPE_BF16 && d->dtype != POPE_F16)
    return fail(POPE_ERR_UNSUPPORTED, "flash kernels take bf16 or fp16 (dtype %d)", d->dtype);
  if (d->D > kFlashWideMaxD)
    return fail(POPE_ERR_UNSUPPORTED, "flash kernels cover head dim <= %d (got %d)", kFlashWideMaxD, d->D);
  if (!q || !k || !v || !o || !lse) return fail(POPE_ERR_INVALID, "q, k, v, o and lse must be non-NULL");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(POPE_ERR_INVALID, "q, k, v, o must be 16-byte aligned");
  if ((rc = check_strides16("q", d->q_s)) || (rc = check_strides16("k", d->k_s)) ||
      (rc = check_strides16("v", d->v_s)) || (rc = check_strides16("o", d->o_s)))
    return rc;
  if ((rc = check_pope_ptrs(d, freqs, bias))) return rc;
  if (d->mask_sb < 0) return fail(POPE_ERR_INVALID, "negative mask stride");
  (void)mask;
  if (d->softmax_scale != d->softmax_scale) return fail(POPE_ERR_INVALID, "softmax scale is NaN");
  return POPE_OK;
}


// op_flags: the flags one entry point accepts beyond SPLIT_BF16 and DETERMINISTIC.
int check_sim_common(const pope_desc* d, const void* q, const void* k, const float* freqs, const float* bias,
                     unsigned op_flags) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (d->dtype != POPE_F32) return fail(POPE_ERR_UNSUPPORTED, "similarity kernels take fp32 (dtype %d)", d->dtype);
  if (d->flags & ~(POPE_FLAG_SPLIT_BF16 | POPE_FLAG_DETERMINISTIC | op_flags))
    return fail(POPE_ERR_INVALID, "unknown flags 0x%x", (unsigned)d->flags);
  if (d->D > 512) return fail(POPE_ERR_UNSUPPORTED, "similarity covers head dim <= 512 (got %d)", d->D);
  if (!q || !k) return fail(POPE_ERR_INVALID, "q, k must be non-NULL");
  if (!aligned16(q) || !aligned16(k)) return fail(POPE_ERR_INVALID, "q, k must be 16-byte aligned");
  if ((rc = check_strides32("q", d->q_s)) || (rc = check_strides32("k", d->k_s))) return rc;
  return check_pope_ptrs(d, freqs, bias);
}

// Builds the key table (with bias) and the query table (without) for the fp32 kernels (the
// split-bf16 kernels compute the phases in place) and fills the shared parameters.
hipError_t sim_setup(const pope_desc& d, const void* q, const void* k, const float* freqs, const float* bias,
                     char* ws, hipStream_t s, pope::SimParams* out) {
  pope::SimParams& p = *out;
  std::memset(&p, 0, sizeof p);
  const int Bt = d.f_s[0] != 0 ? d.B : 1;
  const int Hqt = d.f_s[1] != 0 ? d.Hq : 1;
  float2* ktab = reinterpret_cast<float2*>(ws);
  float2* qtab = reinterpret_cast<float2*>(ws + sim_table_k(d));
  // the fp32 kernels read the phases from tables; the split-bf16 kernels compute them in place
  const bool tables = d.R > 0 && !(d.flags & POPE_FLAG_SPLIT_BF16);
  if (tables) {
    hipError_t e = build_table(d, freqs, bias, Bt, d.Hk, ktab, s);
    if (e != hipSuccess) return e;
    e = build_table(d, freqs, nullptr, Bt, Hqt, qtab, s);  // query phases never carry the bias
    if (e != hipSuccess) return e;
  }
  p.q = static_cast<const float*>(q);
  p.k = static_cast<const float*>(k);
  p.freqs = d.R > 0 ? freqs : nullptr;
  p.bias = d.R > 0 ? bias : nullptr;
  p.ktab = tables ? ktab : nullptr;
  p.qtab = tables ? qtab : nullptr;
  p.B = d.B; p.Hq = d.Hq; p.Hk = d.Hk; p.Nq = d.Nq; p.Nk = d.Nk; p.D = d.D; p.R = d.R;
  p.E = d.D + d.R;
  p.EP = round_up(p.E, 32);
  copy3(p.q_s, d.q_s);
  copy3(p.k_s, d.k_s);
  copy3(p.sim_s, d.sim_s);
  copy3(p.f_s, d.f_s);
  p.bias_sh = d.bias_sh;
  p.kt_sb = Bt > 1 ? (int64_t)d.Hk * d.Nk * d.R : 0;
  p.kt_sh = (int64_t)d.Nk * d.R;
  p.qt_sb = Bt > 1 ? (int64_t)Hqt * d.Nk * d.R : 0;
  p.qt_sh = Hqt > 1 ? (int64_t)d.Nk * d.R : 0;
  return hipSuccess;
}

}  // namespace

extern "C" {

int pope_abi_version(void) { return POPE_ABI_VERSION; }

int pope_profile_enable(int on) {
  pope::prof_enable(on);
  return POPE_OK;
}

int pope_profile_read(char* buf, size_t n) {
  if (!buf || n == 0) return fail(POPE_ERR_INVALID, "profile buffer is NULL");
  const int rc = pope::prof_read(buf, n);
  if (rc == 1) return fail(POPE_ERR_HIP, "waiting for profiling events failed");
  if (rc == 2) return fail(POPE_ERR_INVALID, "profile buffer of %zu bytes too small", n);
  return POPE_OK;
}

int pope_profile_reset(void) {
  pope::prof_reset();
  return POPE_OK;
}

int pope_last_error(char* buf, size_t n) {
  if (!buf || n == 0) return POPE_ERR_INVALID;
  std::strncpy(buf, g_err.c_str(), n - 1);
  buf[n - 1] = '\0';
  return POPE_OK;
}

int pope_workspace_bytes(int op, const pope_desc* desc, size_t* bytes) {
  if (!bytes) return fail(POPE_ERR_INVALID, "bytes is NULL");
  int rc = check_desc(desc);
  if (rc) return rc;
  switch (op) {
    case POPE_OP_SIM_FWD:
    case POPE_OP_SIM_BWD: *bytes = sim_ws(*desc, op); return POPE_OK;
    case POPE_OP_FLASH_FWD:
    case POPE_OP_FLASH_BWD: *bytes = flash_ws(*desc, op); return POPE_OK;
    case POPE_OP_FLASH_DECODE: *bytes = decode_ws(*desc); return POPE_OK;
    case POPE_OP_POLAR_BWD: *bytes = det_bytes(*desc); return POPE_OK;
    default: return fail(POPE_ERR_INVALID, "unknown op %d", op);
  }
}

int pope_flash_fwd(const pope_desc* d, const void* q, const void* k, const void* v, const float* freqs,
                   const float* bias, const uint8_t* mask, void* o, float* lse, void* workspace,
                   size_t workspace_bytes, void* stream) {
  int rc = check_flash_common(d, q, k, v, freqs, bias, mask, o, lse);
  if (rc) return rc;
  const FlashLayout L = flash_layout(*d);
  if ((rc = check_ws(L.total, workspace, workspace_bytes))) return rc;
  if ((rc = check_row_span("v", L.NkP, d->v_s[2]))) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  hipError_t e = flash_prepare(*d, L, q, k, freqs, bias, mask, ws, s);
  if (e != hipSuccess) return hip_fail(e, "flash preparation launch");
  pope::FlashFwdParams p;
  std::memset(&p, 0, sizeof p);
  p.qh = reinterpret_cast<const uint16_t*>(ws + L.qh);
  p.kh = reinterpret_cast<const uint16_t*>(ws + L.kh);
  p.v = static_cast<const uint16_t*>(v);
  p.mwords = reinterpret_cast<const uint64_t*>(ws + L.mwords);
  p.kend = reinterpret_cast<const int*>(ws + L.kend);
  p.o = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.B = d->B; p.Hq = d->Hq; p.Hk = d->Hk; p.Nq = d->Nq; p.Nk = d->Nk; p.D = d->D;
  p.EP = L.EP; p.DV = L.DV; p.NqP = L.NqP; p.NkP = L.NkP; p.NW = L.NW;
  p.causal = d->causal != 0;
  p.nqb = (d->Nq + 127) / 128;
  copy3(p.v_s, d->v_s);
  copy3(p.o_s, d->o_s);
  e = L.wide ? pope::launch_flash_wide_fwd(p, d->dtype, s) : pope::launch_flash_fwd(p, d->dtype, s);
  if (e == hipErrorInvalidValue)
    return fail(POPE_ERR_UNSUPPORTED, "no flash forward kernel for head dim %d, rotate dim %d", d->D, d->R);
  if (e != hipSuccess) return hip_fail(e, "flash forward launch");
  return POPE_OK;
}

int pope_flash_bwd(const pope_desc* d, const void* dout, const void* q, const void* k, const void* v,
                   const void* o, const float* lse, const float* freqs, const float* bias, const uint8_t* mask,
                   void* dq, void* dk, void* dv, float* dfreqs, float* dbias, void* workspace,
                   size_t workspace_bytes, void* stream) {
  int rc = check_flash_common(d, q, k, v, freqs, bias, mask, o, lse);
  if (rc) return rc;
  if (!dout || !dq || !dk || !dv) return fail(POPE_ERR_INVALID, "dout, dq, dk, dv must be non-NULL");
  if (!aligned16(dout) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
    return fail(POPE_ERR_INVALID, "dout, dq, dk, dv must be 16-byte aligned");
  if ((rc = check_strides16("do", d->do_s)) || (rc = check_strides16("dq", d->dq_s)) ||
      (rc = check_strides16("dk", d->dk_s)) || (rc = check_strides16("dv", d->dv_s)))
    return rc;
  if (d->R == 0 && (dfreqs || dbias)) return fail(POPE_ERR_INVALID, "dfreqs/dbias requested with rotate dim 0");
  if (d->flags & ~(POPE_FLAG_PREPARED | POPE_FLAG_ZERO_GRADS | POPE_FLAG_DETERMINISTIC))
    return fail(POPE_ERR_INVALID, "unknown flags 0x%x", (unsigned)d->flags);
  const FlashLayout L = flash_layout(*d);
  if ((rc = check_ws(L.total + L.wide_bytes + det_bytes(*d), workspace, workspace_bytes))) return rc;
  if ((rc = check_row_span("v", L.NkP, d->v_s[2])) || (rc = check_row_span("do", L.NqP, d->do_s[2]))) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (!(d->flags & POPE_FLAG_PREPARED)) {
    hipError_t e = flash_prepare(*d, L, q, k, freqs, bias, mask, ws, s);
    if (e != hipSuccess) return hip_fail(e, "flash preparation launch");
  }
  pope::FlashBwdParams p;
  std::memset(&p, 0, sizeof p);
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<const uint16_t*>(o);
  p.dout = static_cast<const uint16_t*>(dout);
  p.lse = lse;
  p.mask = mask;
  p.table = d->R > 0 ? reinterpret_cast<const float2*>(ws + L.table) : nullptr;
  p.btab = d->R > 0 ? reinterpret_cast<const float2*>(ws + L.btab) : nullptr;
  p.dq = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.dfreqs = dfreqs;
  p.dbias = dbias;
  p.qh = reinterpret_cast<const uint16_t*>(ws + L.qh);
  p.kh = reinterpret_cast<const uint16_t*>(ws + L.kh);
  p.nl = reinterpret_cast<float*>(ws + L.ld);
  p.nd = p.nl + (size_t)d->B * d->Hq * L.NqP;
  p.mwords = reinterpret_cast<const uint64_t*>(ws + L.mwords);
  p.kend = reinterpret_cast<const int*>(ws + L.kend);
  p.NW = L.NW;
  p.B = d->B; p.Hq = d->Hq; p.Hk = d->Hk; p.Nq = d->Nq; p.Nk = d->Nk; p.D = d->D; p.R = d->R;
  p.E = d->D + d->R;
  p.EP = L.EP;
  p.DV = L.DV;
  p.NqP = L.NqP;
  p.NkP = L.NkP;
  p.Bt = L.Bt; p.Ht = L.Ht; p.Hb = L.Hb;
  p.causal = d->causal != 0;
  p.has_mask = mask != nullptr;
  p.zero_grads = (d->flags & POPE_FLAG_ZERO_GRADS) != 0;
  p.scale = d->softmax_scale;
  copy3(p.q_s, d->q_s); copy3(p.k_s, d->k_s); copy3(p.v_s, d->v_s);
  copy3(p.o_s, d->o_s); copy3(p.do_s, d->do_s); copy3(p.dq_s, d->dq_s);
  copy3(p.dk_s, d->dk_s); copy3(p.dv_s, d->dv_s);
  copy3(p.df_s, d->df_s);
  p.bias_sh = d->bias_sh;
  p.mask_sb = d->mask_sb;
  p.t_sb = L.Bt > 1 ? (int64_t)L.Ht * d->Nk * d->R : 0;
  p.t_sh = L.Ht > 1 ? (int64_t)d->Nk * d->R : 0;
  const DetParts dp = det_parts(*d, ws + L.total + L.wide_bytes, dfreqs, dbias);
  p.kpart = dp.kpart;
  p.qpart = dp.qpart;
  hipError_t e;
  if (L.wide) {
    e = pope::launch_flash_bwd_delta(p, d->dtype, s);
    if (e == hipSuccess)
      e = pope::launch_flash_wide_bwd(p, reinterpret_cast<float*>(ws + L.wk), reinterpret_cast<float*>(ws + L.wq),
                                      d->dtype, s);
  } else {
    e = pope::launch_flash_bwd(p, d->dtype, s);
  }
  if (e == hipErrorInvalidValue)
    return fail(POPE_ERR_UNSUPPORTED, "no flash backward kernel for head dim %d, rotate dim %d", d->D, d->R);
  if (e != hipSuccess) return hip_fail(e, "flash backward launch");
  e = det_reduce(*d, dp, dfreqs, dbias, (d->flags & POPE_FLAG_ZERO_GRADS) != 0, s);
  if (e != hipSuccess) return hip_fail(e, "phase gradient reduction launch");
  return POPE_OK;
}

int pope_flash_decode(const pope_desc* d, const void* q, const void* k, const void* v, const float* freqs,
                      const float* bias, const uint8_t* mask, void* o, float* lse, void* workspace,
                      size_t workspace_bytes, void* stream) {
  int rc = check_flash_common(d, q, k, v, freqs, bias, mask, o, lse);
  if (rc) return rc;
  if (d->Nq != 1 || d->causal || d->D > 128)
    return fail(POPE_ERR_UNSUPPORTED, "decode kernel covers one non-causal query row with head dim <= 128 "
                                      "(got %d rows, causal %d, head dim %d)", d->Nq, d->causal, d->D);
  if (d->R > 0 && d->f_s[1] != 0)
    return fail(POPE_ERR_UNSUPPORTED, "decode kernel: per-head freqs tables are not covered");
  if (pope::decode_head_groups(d->Hq, d->D) == 0)
    return fail(POPE_ERR_UNSUPPORTED, "decode kernel: no power-of-two group of the %d query heads has at most "
                "4096 query-weight words (head dim %d)", d->Hq, d->D);
  // the split kernel reads freqs rows as 16-byte vectors
  if (d->R > 0 && ((reinterpret_cast<uintptr_t>(freqs) & 15u) || d->f_s[0] % 4 || d->f_s[2] % 4))
    return fail(POPE_ERR_UNSUPPORTED, "decode kernel: freqs rows must be 16-byte aligned");
  // the split kernel addresses rows of one (batch, head) with 32-bit element offsets
  if ((int64_t)(d->Nk - 1) * std::max(d->k_s[2], d->v_s[2]) + d->D >= INT32_MAX)
    return fail(POPE_ERR_UNSUPPORTED, "decode kernel: K / V row offsets exceed 32 bits (rows %d, strides %lld, %lld)",
                d->Nk, (long long)d->k_s[2], (long long)d->v_s[2]);
  if ((rc = check_ws(decode_ws(*d), workspace, workspace_bytes))) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const Geo g = geometry(*d, d->Hq);
  char* ws = static_cast<char*>(workspace);
  const int splits = decode_splits(*d);
  const size_t rows = (size_t)d->B * d->Hq * d->Nq;
  float* part_o = reinterpret_cast<float*>(ws);
  float* part_ml = reinterpret_cast<float*>(ws + align_up(rows * splits * d->D * sizeof(float)));
  pope::DecodeParams p;
  std::memset(&p, 0, sizeof p);
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.freqs = d->R > 0 ? freqs : nullptr;
  p.bias = d->R > 0 ? bias : nullptr;
  p.mask = mask;
  p.o = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.part_o = part_o;
  p.part_ml = part_ml;
  p.B = d->B; p.Hq = d->Hq; p.Hk = d->Hk; p.Nq = d->Nq; p.Nk = d->Nk; p.D = d->D; p.R = d->R;
  p.causal = d->causal != 0;
  p.has_mask = mask != nullptr;
  p.splits = splits;
  p.keys_per_split = (d->Nk + splits - 1) / splits;
  p.scale_log2 = d->softmax_scale * 1.4426950408889634f;
  copy3(p.q_s, d->q_s); copy3(p.k_s, d->k_s); copy3(p.v_s, d->v_s);
  copy3(p.o_s, d->o_s); copy3(p.f_s, d->f_s);
  p.bias_sh = d->bias_sh;
  p.mask_sb = d->mask_sb;
  p.t_sb = g.Bt > 1 ? (int64_t)g.Ht * d->Nk * d->R : 0;
  p.t_sh = g.Ht > 1 ? (int64_t)d->Nk * d->R : 0;
  hipError_t e = pope::launch_flash_decode(p, d->dtype, s);
  if (e == hipErrorInvalidValue)
    return fail(POPE_ERR_UNSUPPORTED, "no decode kernel for head dim %d, rotate dim %d", d->D, d->R);
  if (e != hipSuccess) return hip_fail(e, "flash decode launch");
  return POPE_OK;
}

int pope_flash_decode_noalloc(const pope_desc* d, const void* q, const void* k, const void* v,
                              const float* freqs, const float* bias, const uint8_t* mask, void* o, float* lse,
                              void* stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  const size_t need = decode_ws(*d);
  if (need > pope::kDecodeScratchBytes)
    return fail(POPE_ERR_WORKSPACE, "decode without allocation: %zu bytes of split partials exceed the library's "
                "%zu-byte scratch array (fewer batch rows x query heads or a shorter cache fit)",
                need, pope::kDecodeScratchBytes);
  void* ws = nullptr;
  const hipError_t e = pope::decode_scratch(&ws);
  if (e != hipSuccess) return hip_fail(e, "decode scratch address");
  return pope_flash_decode(d, q, k, v, freqs, bias, mask, o, lse, ws, pope::kDecodeScratchBytes, stream);
}

int pope_sim_fwd(const pope_desc* d, const void* q, const void* k, const float* freqs, const float* bias,
                 void* sim, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_sim_common(d, q, k, freqs, bias, 0);
  if (rc) return rc;
  if (!sim) return fail(POPE_ERR_INVALID, "sim must be non-NULL");
  if (d->sim_s[0] < 0 || d->sim_s[1] < 0 || d->sim_s[2] < 0) return fail(POPE_ERR_INVALID, "negative sim stride");
  if ((rc = check_ws(sim_ws(*d, POPE_OP_SIM_FWD), workspace, workspace_bytes))) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  pope::SimParams p;
  hipError_t e = sim_setup(*d, q, k, freqs, bias, static_cast<char*>(workspace), s, &p);
  if (e != hipSuccess) return hip_fail(e, "phase table launch");
  p.sim = static_cast<float*>(sim);
  if (d->flags & POPE_FLAG_SPLIT_BF16)
    e = pope::launch_sim_split_fwd(p, sim_split_planes(*d, static_cast<char*>(workspace), POPE_OP_SIM_FWD), s);
  else
    e = pope::launch_sim_fwd(p, s);
  if (e != hipSuccess) return hip_fail(e, "similarity forward launch");
  return POPE_OK;
}

int pope_sim_bwd(const pope_desc* d, const void* dsim, const void* q, const void* k, const float* freqs,
                 const float* bias, void* dq, void* dk, float* dfreqs, float* dbias, void* workspace,
                 size_t workspace_bytes, void* stream) {
  int rc = check_sim_common(d, q, k, freqs, bias, POPE_FLAG_ZERO_GRADS);
  if (rc) return rc;
  if (!dsim || !dq || !dk) return fail(POPE_ERR_INVALID, "dsim, dq, dk must be non-NULL");
  if (!aligned16(dq) || !aligned16(dk)) return fail(POPE_ERR_INVALID, "dq, dk must be 16-byte aligned");
  if (d->sim_s[0] < 0 || d->sim_s[1] < 0 || d->sim_s[2] < 0) return fail(POPE_ERR_INVALID, "negative dsim stride");
  if ((rc = check_strides32("dq", d->dq_s)) ||
      (rc = check_strides32("dk", d->dk_s)))
    return rc;
  if (d->R == 0 && (dfreqs || dbias)) return fail(POPE_ERR_INVALID, "dfreqs/dbias requested with rotate dim 0");
  if (d->df_s[0] < 0 || d->df_s[1] < 0 || d->df_s[2] < 0) return fail(POPE_ERR_INVALID, "negative dfreqs stride");
  if ((rc = check_ws(sim_ws(*d, POPE_OP_SIM_BWD), workspace, workspace_bytes))) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  pope::SimParams p;
  hipError_t e = sim_setup(*d, q, k, freqs, bias, ws, s, &p);
  if (e != hipSuccess) return hip_fail(e, "phase table launch");
  p.dsim = static_cast<const float*>(dsim);
  // 4-wide loads of dsim rows, addressed with 32-bit offsets within one (batch, head)
  p.g_vec = aligned16(dsim) && d->sim_s[0] % 4 == 0 && d->sim_s[1] % 4 == 0 && d->sim_s[2] % 4 == 0 &&
            (int64_t)d->Nq * d->sim_s[2] < ((int64_t)1 << 31);
  p.dq = static_cast<float*>(dq);
  p.dk = static_cast<float*>(dk);
  p.dfreqs = dfreqs;
  p.dbias = dbias;
  copy3(p.dq_s, d->dq_s);
  copy3(p.dk_s, d->dk_s);
  copy3(p.df_s, d->df_s);
  const size_t off_u = sim_table_k(*d) + sim_table_q(*d);
  float* U = reinterpret_cast<float*>(ws + off_u);
  float* W = reinterpret_cast<float*>(ws + off_u + align_up((size_t)d->B * d->Hq * d->Nq * p.EP * sizeof(float)));
  const DetParts dp = det_parts(*d, ws + sim_ws(*d, POPE_OP_SIM_BWD) - det_bytes(*d), dfreqs, dbias);
  p.kpart = dp.kpart;
  p.qpart = dp.qpart;
  const bool zero = (d->flags & POPE_FLAG_ZERO_GRADS) != 0;
  // deterministic mode: the phase-gradient reduction overwrites dfreqs / dbias instead
  p.zero_grads = zero && !dp.kpart && (dfreqs || dbias);
  p.Bt = d->f_s[0] != 0 ? d->B : 1;
  p.Ht = d->f_s[1] != 0 ? d->Hq : 1;   // per-head tables need Hq == Hk
  p.Hb = d->bias_sh != 0 ? d->Hk : 1;
  if (d->flags & POPE_FLAG_SPLIT_BF16)
    e = pope::launch_sim_split_bwd(p, sim_split_planes(*d, ws, POPE_OP_SIM_BWD), U, W, s);
  else
    e = pope::launch_sim_bwd_ws(p, U, W, s);
  if (e != hipSuccess) return hip_fail(e, "similarity backward launch");
  e = det_reduce(*d, dp, dfreqs, dbias, zero, s);
  if (e != hipSuccess) return hip_fail(e, "phase gradient reduction launch");
  return POPE_OK;
}

}  // extern "C"

namespace {

int check_polar(const pope_desc* d, const void* q, const void* k, const float* freqs, const float* bias) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (d->dtype != POPE_F32 && d->dtype != POPE_F16 && d->dtype != POPE_BF16)
    return fail(POPE_ERR_INVALID, "unknown dtype %d", d->dtype);
  if (d->D > 512) return fail(POPE_ERR_UNSUPPORTED, "polar transform covers head dim <= 512 (got %d)", d->D);
  if (!q || !k) return fail(POPE_ERR_INVALID, "q, k must be non-NULL");
  const size_t al = d->dtype == POPE_F32 ? 16 : 8;
  if (reinterpret_cast<uintptr_t>(q) % al || reinterpret_cast<uintptr_t>(k) % al)
    return fail(POPE_ERR_INVALID, "q, k must be %zu-byte aligned", al);
  for (int i = 0; i < 3; ++i)
    if (d->q_s[i] < 0 || d->q_s[i] % 4 || d->k_s[i] < 0 || d->k_s[i] % 4)
      return fail(POPE_ERR_INVALID, "q / k strides must be non-negative multiples of 4");
  if (d->R > 0 && d->bias_sh != 0 && d->bias_sh < d->R) return fail(POPE_ERR_INVALID, "bias row stride below R");
  if (d->flags & ~(POPE_FLAG_COMPLEX | POPE_FLAG_DETERMINISTIC))
    return fail(POPE_ERR_INVALID, "unknown flags 0x%x", (unsigned)d->flags);
  return check_pope_ptrs(d, freqs, bias);
}

void polar_params(const pope_desc* d, const void* q, const void* k, const float* freqs, const float* bias,
                  pope::PolarParams* p) {
  std::memset(p, 0, sizeof *p);
  p->q = q; p->k = k;
  p->freqs = d->R > 0 ? freqs : nullptr;
  p->bias = d->R > 0 ? bias : nullptr;
  p->B = d->B; p->Hq = d->Hq; p->Hk = d->Hk; p->Nq = d->Nq; p->Nk = d->Nk; p->D = d->D; p->R = d->R;
  p->cplx = (d->flags & POPE_FLAG_COMPLEX) != 0;
  copy3(p->q_s, d->q_s); copy3(p->k_s, d->k_s); copy3(p->f_s, d->f_s);
  p->bias_sh = d->bias_sh;
}

int polar_dtype(const pope_desc* d) { return d->dtype == POPE_F32 ? 0 : d->dtype == POPE_F16 ? 1 : 2; }

}  // namespace

extern "C" {

int pope_polar_fwd(const pope_desc* d, const void* q, const void* k, const float* freqs, const float* bias,
                   float* q_hat, float* k_hat, void* stream) {
  int rc = check_polar(d, q, k, freqs, bias);
  if (rc) return rc;
  if (!q_hat || !k_hat || !aligned16(q_hat) || !aligned16(k_hat))
    return fail(POPE_ERR_INVALID, "q_hat, k_hat must be non-NULL and 16-byte aligned");
  pope::PolarParams p;
  polar_params(d, q, k, freqs, bias, &p);
  p.qh = q_hat; p.kh = k_hat;
  const hipError_t e = pope::launch_polar(p, polar_dtype(d), false, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "polar transform launch");
  return POPE_OK;
}

int pope_polar_bwd(const pope_desc* d, const float* dq_hat, const float* dk_hat, const void* q, const void* k,
                   const float* freqs, const float* bias, void* dq, void* dk, float* dfreqs, float* dbias,
                   void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_polar(d, q, k, freqs, bias);
  if (rc) return rc;
  if (!dq_hat || !dk_hat || !aligned16(dq_hat) || !aligned16(dk_hat))
    return fail(POPE_ERR_INVALID, "dq_hat, dk_hat must be non-NULL and 16-byte aligned");
  const size_t al = d->dtype == POPE_F32 ? 16 : 8;
  if (!dq || !dk || reinterpret_cast<uintptr_t>(dq) % al || reinterpret_cast<uintptr_t>(dk) % al)
    return fail(POPE_ERR_INVALID, "dq, dk must be non-NULL and %zu-byte aligned", al);
  for (int i = 0; i < 3; ++i)
    if (d->dq_s[i] < 0 || d->dq_s[i] % 4 || d->dk_s[i] < 0 || d->dk_s[i] % 4)
      return fail(POPE_ERR_INVALID, "dq / dk strides must be non-negative multiples of 4");
  if (d->R == 0 && (dfreqs || dbias)) return fail(POPE_ERR_INVALID, "dfreqs/dbias requested with rotate dim 0");
  if (d->df_s[0] < 0 || d->df_s[1] < 0 || d->df_s[2] < 0) return fail(POPE_ERR_INVALID, "negative dfreqs stride");
  if ((rc = check_ws(det_bytes(*d), workspace, workspace_bytes))) return rc;
  pope::PolarParams p;
  polar_params(d, q, k, freqs, bias, &p);
  p.gq = dq_hat; p.gk = dk_hat; p.dq = dq; p.dk = dk; p.dfreqs = dfreqs; p.dbias = dbias;
  copy3(p.dq_s, d->dq_s); copy3(p.dk_s, d->dk_s); copy3(p.df_s, d->df_s);
  const DetParts dp = det_parts(*d, static_cast<char*>(workspace), dfreqs, dbias);
  p.kpart = dp.kpart;
  p.qpart = dp.qpart;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = pope::launch_polar(p, polar_dtype(d), true, s);
  if (e != hipSuccess) return hip_fail(e, "polar transform backward launch");
  e = det_reduce(*d, dp, dfreqs, dbias, false, s);
  if (e != hipSuccess) return hip_fail(e, "phase gradient reduction launch");
  return POPE_OK;
}

}  // extern "C"
