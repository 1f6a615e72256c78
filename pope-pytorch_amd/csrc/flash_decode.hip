// Single-query flash attention with PoPE against a long KV cache (gfx950).
//
// Reference semantics: flash_attn_forward at seqlen_q = 1
// (triton_pope_flash_attn.py:222-271, kernel :23-117 with grid (1, B*H)); the
// query phase is freqs[Nk - 1] (q_off = Nk - Nq, :54; pope.py:64).  Non-causal
// (top-left causal with one query sees key 0 only and takes the general
// forward path).
//
// The path is bound by HBM: every valid key costs 2 * D * 2 bytes of K and V
// and a handful of flops.  Work decomposition (two launches):
//   decode_split : one workgroup (4 waves) per (batch, split of S keys, group of query
//                  heads: all of them unless their query weights exceed the LDS array);
//                  wave w takes the group's heads w, w + 4, ...
//                  A split whose keys are all masked exits after reading its mask
//                  bytes.  The workgroup computes its heads' query weights (below)
//                  into LDS, and the cos / sin of its rows of F (fp16 pairs, from the
//                  fp32 rows of the caller's freqs, which every batch's splits read
//                  out of L2), staged in LDS once and shared by all heads.  A wave load reads
//                  64 / LPK consecutive key rows of one head (LPK lanes x 16 bytes per
//                  row), so every wave streams contiguous memory; all K and V rows of a
//                  head are in flight before its scores are computed, and the next
//                  head's rows are loaded while the current head is finished.  Per key:
//                  the polar transform of the key (softplus(k) times the staged cos /
//                  sin) folded with the query's (cos, sin) weights, summed over the
//                  row's lanes; the head's max, sum and p-weighted V rows reduce across
//                  the rows by lane shuffles into one (m, l, o) per (batch, head, split).
//                  Loads are branch-free (clamped addresses), so each wait covers only
//                  the rows being computed.
//   decode_combine : merges the splits of each (batch, head) by their log-sum-exp
//                  and writes o (input dtype) and lse (natural log, -inf when
//                  every key is masked).
// The query weights use the bias-on-the-query-side form of the score,
//   a_d c_jd cos((F_q,d - b_d) - F_j,d)
//     = c_jd [a_d cos(F_q,d - b_d) cos F_j,d + a_d sin(F_q,d - b_d) sin F_j,d],
// so the key side needs only cos / sin(F_j) (shared by every head and batch).
#include <mutex>
#include <type_traits>

#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kThreads = 256;



// Sum over aligned groups of LPK lanes (LPK = 4, 8 or 16) with DPP lane moves (VALU, no LDS
// round trip): xor 1 and xor 2 by quad permutes, then the half-row mirror (lane i <-> 7 - i in
// each 8-lane half) joins the two quads, and a row mirror (i <-> 15 - i) the two halves.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int LPK>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp_move<0xB1>(x);                    // quad_perm [1, 0, 3, 2]
  x += dpp_move<0x4E>(x);                    // quad_perm [2, 3, 0, 1]
  if (LPK >= 8) x += dpp_move<0x141>(x);     // row_half_mirror
  if (LPK >= 16) x += dpp_move<0x140>(x);    // row_mirror
  return x;
}

// Inputs of the query weight word of (batch b, head h, dim d): q, and for a rotated dim F_q and
// the bias.
struct QwIn {
  float qv, f, bb;
};
template <typename T>
__device__ __forceinline__ QwIn query_weight_in(const DecodeParams& p, int b, int h, int d) {
  QwIn in;
  in.qv = T::to_float(p.q[(int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1] + d]);
  in.f = in.bb = 0.f;
  if (d < p.R) {
    in.f = p.freqs[(int64_t)b * p.f_s[0] + (int64_t)(p.Nk - 1) * p.f_s[2] + d];
    in.bb = p.bias[(int64_t)(h % p.Hk) * p.bias_sh + d];
  }
  return in;
}
// The query weight word, scale * log2 e folded in: rotated dims the fp16 pair
// (a cos(F_q - b), a sin(F_q - b)) with a = softplus(q) and F_q = F[Nk - 1]; pass-through dims
// the fp32 weight q.
__device__ __forceinline__ uint32_t query_weight_of(const DecodeParams& p, int d, QwIn in) {
  if (d < p.R) {
    float sn, cs;
    sincos_acc(in.f - in.bb, &sn, &cs);
    const float a = softplus_f(in.qv) * p.scale_log2;
    return __builtin_bit_cast(uint32_t, f16x2{(_Float16)(a * cs), (_Float16)(a * sn)});
  }
  return __builtin_bit_cast(uint32_t, in.qv * p.scale_log2);
}

// Split kernel.  A workgroup (4 waves) owns one (batch, split of S keys) for one group of query
// heads (hgroups groups of Hq / hgroups heads: one group unless the heads' query weights exceed
// kQwMax words); wave w takes the group's heads w, w + 4, ...  Lane = row r * LPK + chunk c: a load instruction of a wave
// reads RPI = 64 / LPK consecutive key rows of one head (LPK lanes x 16 bytes per row), so a
// wave streams contiguous memory, and load u of a head covers keys u * RPI + r.  A head's
// kLoads K rows and kLoads V rows are all in flight before its scores are computed (the V
// loads land while the K side is computed).  Per key: the polar-transform score summed over
// the row's LPK lanes (DPP), masked keys -inf; the head's max, sum and p-weighted V rows are
// reduced across the RPI rows by lane shuffles, and the row-0 lanes write the partial.
constexpr int kLoads = 16;
// Query weight words staged in LDS per workgroup: Hq * D of them (the host sends calls with more
// to the general forward).
constexpr int kQwMax = 4096;

// bf16 keys: log2(1 + 2^(-|x| log2 e)) (the softplus term beyond max(x, 0), in log2 units) is
// tabulated in LDS over the bf16 magnitudes 2^-24 <= |x| < 32, indexed by the 15 magnitude bits
// less kSpLo.  Smaller magnitudes take the first entry (off by < 1e-7), larger ones the last
// (the term is below 2e-14 there).  In range, the entry is the value the formula computes.
constexpr int kSpLo = 103 << 7, kSpN = (132 << 7) - kSpLo;

template <int LPK>
constexpr int split_rows() { return kLoads * (64 / LPK); }

// Sum over the lanes that share a chunk (lane bits above the LPK ones).
template <int LPK>
__device__ __forceinline__ float rows_sum(float x) {
#pragma unroll
  for (int m = LPK; m < 64; m <<= 1) x += __shfl_xor(x, m, 64);
  return x;
}
template <int LPK>
__device__ __forceinline__ float rows_max(float x) {
#pragma unroll
  for (int m = LPK; m < 64; m <<= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
  return x;
}

template <typename T, int LPK, int RMAX>
__global__ __launch_bounds__(kThreads, 2) void decode_split_kernel(DecodeParams p) {
  constexpr int RPI = 64 / LPK;          // key rows per load instruction
  constexpr int S = split_rows<LPK>();   // keys per split
  constexpr int TS = RMAX + 4;           // table row stride (words; 16-byte pad spreads banks)
  __shared__ __attribute__((aligned(16))) uint32_t tab_s[S * TS];
  __shared__ __attribute__((aligned(16))) uint32_t qw_s[kQwMax];
  __shared__ uint8_t vis_s[S];
  __shared__ float sp_s[T::kCode == 2 ? kSpN : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane / LPK, c = lane % LPK;
  const int hg = blockIdx.x % p.hgroups, rest = blockIdx.x / p.hgroups;
  const int split = rest % p.splits, b = rest / p.splits;
  const int HG = p.Hq / p.hgroups, h_lo = hg * HG, h_hi = h_lo + HG;   // the workgroup's query heads
  const int D = p.D, R = p.R, Nk = p.Nk;
  const int d0 = 8 * c;
  const bool cact = d0 < D;
  const bool rot = cact && d0 < R;   // R is a multiple of 8: a chunk is all rotated or all pass-through
  const int j_begin = split * S;
  const int nkeys = min(S, Nk - j_begin);
  const uint8_t* mrow = p.has_mask ? p.mask + (int64_t)b * p.mask_sb : nullptr;

  // ---- key visibility of the split into LDS; skip splits without a visible key ----
  int vis_any = 0;
  for (int j = tid; j < S; j += kThreads) {
    const int v = j < nkeys && (!p.has_mask || mrow[j_begin + j] != 0);
    vis_s[j] = (uint8_t)v;
    vis_any |= v;
  }
  if (!__syncthreads_or(vis_any)) {   // (m, l) = (-inf, 0); the combine never reads o of such a split
    for (int i = tid; i < HG; i += kThreads) {
      const int64_t row = ((int64_t)b * p.Hq + h_lo + i) * p.splits + split;
      *reinterpret_cast<float2*>(p.part_ml + row * 2) = make_float2(-INFINITY, 0.f);
    }
    return;
  }

  // Branch-free loads: every lane reads a valid address (rows past the cache clamp to its last
  // row, chunks past D to the last chunk; their data meet zero weights or are never stored), so
  // the compiler counts them.  Offsets within one (batch, head) fit in 32 bits (host check).
  const int dcl = min(d0, D - 8);
  const int rows_left = Nk - 1 - j_begin - r;
  const int ks2 = (int)p.k_s[2], vs2 = (int)p.v_s[2];
  // LDS byte address of the lane's table chunk in its first row (chunks past R read the last
  // staged chunk: finite values that meet zero weights)
  const uint32_t tab_lane = lds_addr(tab_s + r * TS + min(d0, max(R, 8) - 8));

  constexpr int kWaves = kThreads / 64;
  auto kptr = [&](int h) {
    return p.k + (int64_t)b * p.k_s[0] + (int64_t)(h % p.Hk) * p.k_s[1] + ((j_begin + r) * ks2 + dcl);
  };
  auto vptr = [&](int h) {
    return p.v + (int64_t)b * p.v_s[0] + (int64_t)(h % p.Hk) * p.v_s[1] + ((j_begin + r) * vs2 + dcl);
  };
  // The query weight words of a head: two 16-byte LDS reads at the clamped chunk.
  u32x4 qwc[2];
  auto qwload = [&](int h) {
    const uint32_t a = lds_addr(qw_s + (h - h_lo) * D + dcl);
    qwc[0] = lds_read16_at(a);
    qwc[1] = lds_read16_at(a + 16);
  };
  u32x4 kb[kLoads], vb[kLoads];
  // K and V rows are read once per call: non-temporal loads keep them from evicting what is read
  // again (the split's freqs rows, shared by every batch, and the partials the combine reads)
  auto load = [&](u32x4* buf, const uint16_t* lp, int stride) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u)
      buf[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(lp + min(u * RPI, rows_left) * stride));
  };

  // ---- the split's phase rows F[j] (rows past Nk repeat the last row), then the first head's
  // K and V rows, all issued before the rows' (cos, sin) are computed and stored to LDS as fp16
  // pairs: the K / V loads do not wait for that round trip.  Waves past the group's heads load a valid head and
  // never use it.  The rows of the freqs table are read by every batch's splits (L2 hits after
  // the first): no table is built beforehand.
  constexpr int C4 = RMAX / 4;                        // 16-byte chunks per staged row
  constexpr int kTabIt = S * C4 / kThreads;           // chunks per thread
  static_assert(S * C4 % kThreads == 0, "whole table chunks per thread");
  // the first kQwPre query-weight words of each thread: their inputs are loaded with the table
  // rows, so their latency is not exposed after the rows' sine / cosine
  constexpr int kQwPre = 4;
  QwIn qin[kQwPre];
#pragma unroll
  for (int k = 0; k < kQwPre; ++k) {
    const int i = tid + k * kThreads;
    if (i < HG * D) qin[k] = query_weight_in<T>(p, b, h_lo + i / D, i % D);
  }
  float4 tb[kTabIt];
  if (R) {
    const float* fsrc = p.freqs + (int64_t)b * p.f_s[0];
#pragma unroll
    for (int it = 0; it < kTabIt; ++it) {
      const int i = tid + it * kThreads;
      const int c4 = min(i % C4, R / 4 - 1), jj = min(j_begin + i / C4, Nk - 1);
      tb[it] = *reinterpret_cast<const float4*>(fsrc + (int64_t)jj * p.f_s[2] + 4 * c4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const int h0 = min(h_lo + wave, h_hi - 1);
  load(kb, kptr(h0), ks2);
  __builtin_amdgcn_sched_barrier(0);
  load(vb, vptr(h0), vs2);
  __builtin_amdgcn_sched_barrier(0);
  if (R) {
#pragma unroll
    for (int it = 0; it < kTabIt; ++it) {
      const int i = tid + it * kThreads;
      if (i % C4 < R / 4) {
        const float x[4] = {tb[it].x, tb[it].y, tb[it].z, tb[it].w};
        u32x4 w;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float sn, cs;
          sincos_rev(x[t], &sn, &cs);
          w[t] = __builtin_bit_cast(uint32_t, f16x2{(_Float16)cs, (_Float16)sn});
        }
        *reinterpret_cast<u32x4*>(tab_s + (i / C4) * TS + 4 * (i % C4)) = w;
      }
    }
  }
  // query weights of the workgroup's heads (after the rows: their registers are free again)
#pragma unroll
  for (int k = 0; k < kQwPre; ++k) {
    const int i = tid + k * kThreads;
    if (i < HG * D) qw_s[i] = query_weight_of(p, i % D, qin[k]);
  }
  for (int i = tid + kQwPre * kThreads; i < HG * D; i += kThreads)
    qw_s[i] = query_weight_of(p, i % D, query_weight_in<T>(p, b, h_lo + i / D, i % D));
  if constexpr (T::kCode == 2) {
    for (int i = tid; i < kSpN; i += kThreads) {
      const float t = __builtin_bit_cast(float, (uint32_t)(i + kSpLo) << 16);
      sp_s[i] = __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-t * kLog2e));
    }
  }
  __syncthreads();

  // Head h of this wave; with `next` the K rows of head h + kWaves are loaded as soon as the K
  // side of h is done and its V rows as soon as the V side is (the last head of the wave,
  // taken without, loads nothing more).
  auto head = [&](int h, auto next) {
    constexpr bool kNext = decltype(next)::value;

    // query weight words of this lane's 8 dims (zero past D): rotated dims an fp16 pair for
    // v_dot2 with the (cos, sin) table pair, pass-through dims an fp32 weight
    uint32_t wq[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) wq[q] = cact ? qwc[q >> 2][q & 3] : 0u;

    // ---- scores (log2 units) of the lane's kLoads keys ---------------------------------
    float sc[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      float part = 0.f;
      if (R == D || rot) {
        // softplus(x) = max(x, 0) + ln 2 log2(1 + 2^(-|x| log2 e)), the max taken on the bit
        // pattern (x >= 0 iff its signed bits are)
        const uint32_t ta = tab_lane + 4 * TS * RPI * u;
        const u32x4 t0 = lds_read16_at(ta), t1 = lds_read16_at(ta + 16);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t w = kb[u][q >> 1];
          const uint32_t xb = T::kCode == 2 ? ((q & 1) ? (w & 0xffff0000u) : (w << 16))
                                            : __builtin_bit_cast(uint32_t, T::to_float((uint16_t)((q & 1) ? (w >> 16) : (w & 0xffffu))));
          float lt;
          if constexpr (T::kCode == 2) {
            lt = sp_s[min(max((int)((xb >> 16) & 0x7fffu) - kSpLo, 0), kSpN - 1)];
          } else {
            lt = __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-fabsf(__builtin_bit_cast(float, xb)) * kLog2e));
          }
          const float sp = fmaf(lt, kLn2, __builtin_bit_cast(float, max((int)xb, 0)));
          const f16x2 cs = __builtin_bit_cast(f16x2, q < 4 ? t0[q] : t1[q - 4]);
          part = fmaf(sp, __builtin_amdgcn_fdot2(cs, __builtin_bit_cast(f16x2, wq[q]), 0.f, false), part);
        }
      } else {
        float x[8];
        unpack8<T>(kb[u], x);
#pragma unroll
        for (int q = 0; q < 8; ++q) part = fmaf(__builtin_bit_cast(float, wq[q]), x[q], part);
      }
      part = group_sum<LPK>(part);
      sc[u] = vis_s[u * RPI + r] ? part : -INFINITY;
    }
    // keep each group of loads where it is issued (the scheduler would otherwise interleave them
    // with the other group and the waits would cover both)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kNext) {
      qwload(h + kWaves);
      load(kb, kptr(h + kWaves), ks2);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- softmax over the split for this head, o = sum p v -------------------------------
    float m = sc[0];
#pragma unroll
    for (int u = 1; u < kLoads; ++u) m = fmaxf(m, sc[u]);
    m = rows_max<LPK>(m);
    const float mu = m == -INFINITY ? 0.f : m;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const float pv = __builtin_amdgcn_exp2f(sc[u] - mu);   // 0 when masked
      float x[8];
      unpack8<T>(vb[u], x);
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = fmaf(pv, x[q], acc[q]);
      l += pv;
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kNext) load(vb, vptr(h + kWaves), vs2);
    __builtin_amdgcn_sched_barrier(0);
    l = rows_sum<LPK>(l);   // every lane of a row group holds the same p: one lane per row counts
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = rows_sum<LPK>(acc[q]);
    const int64_t row = ((int64_t)b * p.Hq + h) * p.splits + split;
    if (r == 0 && cact) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (d0 + q < D) p.part_o[row * D + d0 + q] = acc[q];
    }
    if (lane == 0) {
      p.part_ml[row * 2] = m;
      p.part_ml[row * 2 + 1] = l;
    }
  };
  if (h_lo + wave < h_hi) {
    int h = h_lo + wave;
    qwload(h);
    for (; h + kWaves < h_hi; h += kWaves) head(h, std::true_type{});
    head(h, std::false_type{});
  }
}

// One workgroup per (batch, head): merge the splits by log-sum-exp.  Thread = (split group g,
// 4-dim quad q); group g takes every G-th split, eight splits' (m, l, o) loads in flight at a
// time, and keeps a running (m, l, o) of its splits (one pass over the partials, no wait for a
// global maximum first); the groups' states then merge through LDS.
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams p) {
  __shared__ float4 o_s[256];
  __shared__ float2 ml_s[256];
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int b = bh / p.Hq, h = bh % p.Hq;
  const int D = p.D, S = p.splits;
  const float2* pml = reinterpret_cast<const float2*>(p.part_ml) + (int64_t)bh * S;
  const float* po = p.part_o + (int64_t)bh * S * D;
  const int qd = D / 4, G = 256 / qd;
  const int g = tid / qd, q = tid % qd;
  float m = -INFINITY, l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  // folds one split into the running state; a split without a visible key has m = -inf, l = 0
  // and an o the split kernel never wrote, and leaves the state as it is
  auto fold = [&](float2 ml, float4 v) {
    if (ml.x == -INFINITY) v = make_float4(0.f, 0.f, 0.f, 0.f);
    const float mn = fmaxf(m, ml.x);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float a = __builtin_amdgcn_exp2f(m - mu), w = __builtin_amdgcn_exp2f(ml.x - mu);
    acc.x = fmaf(acc.x, a, v.x * w);
    acc.y = fmaf(acc.y, a, v.y * w);
    acc.z = fmaf(acc.z, a, v.z * w);
    acc.w = fmaf(acc.w, a, v.w * w);
    l = fmaf(l, a, ml.y * w);
    m = mn;
  };
  if (g < G) {
    const float4* po4 = reinterpret_cast<const float4*>(po) + q;
    int s = g;
    for (; s + 7 * G < S; s += 8 * G) {
      float2 ml[8];
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        ml[u] = pml[s + u * G];
        v[u] = po4[(int64_t)(s + u * G) * qd];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) fold(ml[u], v[u]);
    }
    for (; s < S; s += G) fold(pml[s], po4[(int64_t)s * qd]);
  }
  o_s[tid] = acc;
  ml_s[tid] = make_float2(m, l);
  __syncthreads();
  if (tid < qd) {
    float M = -INFINITY;
    for (int g2 = 0; g2 < G; ++g2) M = fmaxf(M, ml_s[g2 * qd + tid].x);
    const float Mu = M == -INFINITY ? 0.f : M;
    float L = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int g2 = 0; g2 < G; ++g2) {
      const float2 st = ml_s[g2 * qd + tid];
      const float w = __builtin_amdgcn_exp2f(st.x - Mu);
      const float4 v = o_s[g2 * qd + tid];
      o.x = fmaf(v.x, w, o.x); o.y = fmaf(v.y, w, o.y); o.z = fmaf(v.z, w, o.z); o.w = fmaf(v.w, w, o.w);
      L = fmaf(st.y, w, L);
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint16_t* orow = p.o + (int64_t)b * p.o_s[0] + (int64_t)h * p.o_s[1] + 4 * tid;
    orow[0] = T::bits(o.x * inv);
    orow[1] = T::bits(o.y * inv);
    orow[2] = T::bits(o.z * inv);
    orow[3] = T::bits(o.w * inv);
    if (tid == 0) p.lse[bh] = L > 0.f ? (M + __builtin_amdgcn_logf(L)) * kLn2 : -INFINITY;
  }
}

template <typename T, int LPK, int RMAX>
hipError_t launch_t(const DecodeParams& p0, hipStream_t s) {
  DecodeParams p = p0;
  p.hgroups = decode_head_groups(p.Hq, p.D);
  hipError_t e = launch_named("flash_decode_split", decode_split_kernel<T, LPK, RMAX>,
                              dim3(p.B * p.splits * p.hgroups), dim3(kThreads), s, p);
  if (e != hipSuccess) return e;
  return launch_named("flash_decode_combine", decode_combine_kernel<T>, dim3(p.B * p.Hq), dim3(256), s, p);
}

template <typename T>
hipError_t dispatch(const DecodeParams& p, hipStream_t s) {
  const int chunks = p.D / 8;
  if (chunks <= 4) return launch_t<T, 4, 32>(p, s);
  if (chunks <= 8) return launch_t<T, 8, 64>(p, s);
  if (chunks <= 16) return p.R <= 64 ? launch_t<T, 16, 64>(p, s) : launch_t<T, 16, 128>(p, s);
  return hipErrorInvalidValue;
}

}  // namespace

// ---- the decode's own scratch memory, for callers that cannot allocate --------------------------
//
// One array per GPU the library runs on, held until the process ends.  In host code `scratch`
// names a host-side stand-in, never the device memory: its device address comes from
// hipGetSymbolAddress, asked once per device with that device current, and only that address
// reaches kernels.  Every call on a GPU shares its array (calls that overlap on one GPU race);
// the decode writes every partial it reads in the same call, so nothing must start at zero.
namespace {
static __device__ __align__(256) char scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];
}  // namespace

hipError_t decode_scratch(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

int decode_split_keys(int D) {
  const int chunks = (D + 7) / 8;
  return chunks <= 4 ? split_rows<4>() : chunks <= 8 ? split_rows<8>() : split_rows<16>();
}

int decode_head_groups(int Hq, int D) {
  for (int g = 1; g <= Hq; g *= 2)
    if (Hq % g == 0 && (Hq / g) * D <= kQwMax) return g;
  return 0;
}

hipError_t launch_flash_decode(const DecodeParams& p, int dtype, hipStream_t s) {
  // per-head phase tables would need a table chunk per head: the general forward covers them
  if (p.Nq != 1 || p.causal || p.D > 128 || p.t_sh != 0 || decode_head_groups(p.Hq, p.D) == 0)
    return hipErrorInvalidValue;
  return dtype == 2 ? dispatch<BF16>(p, s) : dispatch<F16>(p, s);
}

}  // namespace pope
