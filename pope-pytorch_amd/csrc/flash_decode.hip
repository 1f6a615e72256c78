// Single-query flash attention with PoPE against a long KV cache (gfx950).
//
// Reference semantics: flash_attn_forward at seqlen_q = 1
// (triton_pope_flash_attn.py:222-271, kernel :23-117 with grid (1, B*H)); the
// query phase is freqs[Nk - 1] (q_off = Nk - Nq, :54; pope.py:64).  Non-causal
// (top-left causal with one query sees key 0 only and takes the general
// forward path).
//
// The path is bound by HBM: every valid key costs 2 * D * 2 bytes of K and V
// and a handful of flops.  Work decomposition:
//   decode_setup : the fp16 cos / sin(F_j) table of the keys and each (batch,
//                  head)'s query weights (below), once per call;
//   decode_split : one workgroup (4 waves) per (batch, split of kSplit keys),
//                  covering every query head of the batch.  A split whose keys
//                  are all masked exits after reading its mask bytes.  The split's
//                  rows of the cos / sin(F_j) table (fp16 pairs) are staged in LDS
//                  once and shared by all heads.  LPK lanes share one key row of
//                  one head (16 bytes each, coalesced); a thread streams every
//                  KP-th key of the split for its head.  Pass 1 streams K: the
//                  polar transform of the key (softplus(k) times the staged cos /
//                  sin) folded with the query's (cos, sin) weights, reduced
//                  across the LPK lanes, scaled scores to LDS.  Pass 2 takes each
//                  head's max over the split and streams V, accumulating p * v.
//                  In both passes the loads of the next batch of keys are issued
//                  before the current batch is computed; the loads are branch-free and the
//                  batch loops uniform, so each wait covers only the batch being computed.
//                  With every dim rotated (R == D) the scores run without per-key branches.  The KP partial states
//                  of a head merge through LDS into one (m, l, o) per (batch,
//                  head, split).
//   decode_combine : merges the splits of each (batch, head) by their log-sum-exp
//                  and writes o (input dtype) and lse (natural log, -inf when
//                  every key is masked).
// The query weights use the bias-on-the-query-side form of the score,
//   a_d c_jd cos((F_q,d - b_d) - F_j,d)
//     = c_jd [a_d cos(F_q,d - b_d) cos F_j,d + a_d sin(F_q,d - b_d) sin F_j,d],
// so the key side needs only cos / sin(F_j) (shared by every head and batch).
#include <type_traits>

#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kThreads = 256;
constexpr int kSplit = 128;    // keys per split (one workgroup)
constexpr int kMaxHG = 16;     // query heads per pass of a workgroup
constexpr int kBatch = 4;      // keys per batch (loads issued together)
constexpr int kMaxR = 128;

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ float2 half2f(uint32_t w) {
  const f16x2 v = __builtin_bit_cast(f16x2, w);
  return make_float2((float)v[0], (float)v[1]);
}

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

// Setup: the fp16 (cos, sin) table of F[bt, n, d] for n < Nk, and each (batch, head)'s query
// weights (scale * log2 e folded in): rotated dims (a cos(F_q - b), a sin(F_q - b)) with
// a = softplus(q) and F_q = F[Nk - 1]; pass-through dims (q, 0).
template <typename T>
__global__ __launch_bounds__(256) void decode_setup_kernel(DecodeParams p, int tab_blocks, int64_t n_tab) {
  if ((int)blockIdx.x < tab_blocks) {
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < n_tab; idx += (int64_t)tab_blocks * 256) {
      const int d = (int)(idx % p.R);
      const int64_t rest = idx / p.R;
      const int n = (int)(rest % p.Nk), bt = (int)(rest / p.Nk);
      float sn, cs;
      sincos_acc(p.freqs[(int64_t)bt * p.f_s[0] + (int64_t)n * p.f_s[2] + d], &sn, &cs);
      const f16x2 v = {(_Float16)cs, (_Float16)sn};
      p.table[idx] = __builtin_bit_cast(uint32_t, v);
    }
    return;
  }
  const int idx = ((int)blockIdx.x - tab_blocks) * 256 + threadIdx.x;
  if (idx >= p.B * p.Hq * p.D) return;
  const int d = idx % p.D, bh = idx / p.D;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const float qv = T::to_float(p.q[(int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1] + d]);
  float2 w;
  if (d < p.R) {
    float sn, cs;
    sincos_acc(p.freqs[(int64_t)b * p.f_s[0] + (int64_t)(p.Nk - 1) * p.f_s[2] + d] - p.bias[(int64_t)hk * p.bias_sh + d],
               &sn, &cs);
    const float a = softplus_f(qv) * p.scale_log2;
    w = make_float2(a * cs, a * sn);
  } else {
    w = make_float2(qv * p.scale_log2, 0.f);
  }
  p.qw[idx] = w;
}

// Thread layout: t = c + LPK * (hl + HG * kp): c = 8-dim chunk of the head dim, hl =
// head within the pass, kp = key parity (the thread streams keys kp, kp + KP, ...).
template <typename T, int LPK, int RMAX>
__global__ __launch_bounds__(kThreads, 2) void decode_split_kernel(DecodeParams p, int HG, int KP) {
  // fp16 (cos, sin) per dim; rows padded by 16 bytes so the key groups of a wave start on
  // different banks
  constexpr int TS = RMAX + 4;
  __shared__ __attribute__((aligned(16))) uint32_t tab_s[kSplit * TS];
  __shared__ float s_lds[kMaxHG][kSplit];
  __shared__ float red_o[kThreads][8];
  __shared__ float red_ml[kThreads / LPK][2];
  __shared__ uint8_t vis_s[kSplit];

  const int tid = threadIdx.x;
  const int split = blockIdx.x % p.splits;
  const int b = blockIdx.x / p.splits;
  const int D = p.D, R = p.R, Nk = p.Nk;
  const int c = tid % LPK, rest = tid / LPK, hl = rest % HG, kp = rest / HG;
  const bool active = kp < KP;
  const int d0 = 8 * c;
  const bool cact = active && d0 < D;
  const bool rot = cact && d0 < R;   // R is a multiple of 8: a chunk is all rotated or all pass-through
  const int j_begin = split * kSplit;
  const int nkeys = min(kSplit, Nk - j_begin);
  const uint8_t* mrow = p.has_mask ? p.mask + (int64_t)b * p.mask_sb : nullptr;

  // ---- key visibility of the split into LDS; skip splits without a visible key ----
  int vis_any = 0;
  for (int j = tid; j < kSplit; j += kThreads) {
    const int v = j < nkeys && (!p.has_mask || mrow[j_begin + j] != 0);
    vis_s[j] = (uint8_t)v;
    vis_any |= v;
  }
  if (!__syncthreads_or(vis_any)) {
    for (int i = tid; i < p.Hq * (D + 2); i += kThreads) {
      const int h = i / (D + 2), e = i % (D + 2);
      const int64_t row = ((int64_t)b * p.Hq + h) * p.splits + split;
      if (e < D) p.part_o[row * D + e] = 0.f;
      else p.part_ml[row * 2 + (e - D)] = e == D ? -INFINITY : 0.f;
    }
    return;
  }

  // ---- stage the split's table rows (rows past Nk repeat the last row) ---------
  if (R) {
    const uint32_t* tsrc = p.table + (int64_t)b * p.t_sb;
    const int n4 = kSplit * R / 4;
    for (int i = tid; i < n4; i += kThreads) {
      const int r = i / (R / 4), c4 = i % (R / 4);
      const int jj = min(j_begin + r, Nk - 1);
      *reinterpret_cast<u32x4*>(tab_s + r * TS + 4 * c4) = reinterpret_cast<const u32x4*>(tsrc + (int64_t)jj * R)[c4];
    }
  }
  __syncthreads();

  // batches per thread, the same for every lane (uniform loops, so the loads can be counted) and
  // even (the loops below take batches in pairs); keys past the split score -inf
  int nbu = (nkeys + KP * kBatch - 1) / (KP * kBatch);
  nbu = max(2, nbu + (nbu & 1));
  // keys of a batch past the split end read clamped rows and score -inf (vis_s = 0)
  for (int hg0 = 0; hg0 < p.Hq; hg0 += HG) {
    const int h = hg0 + hl;
    const bool hact = active && h < p.Hq;
    const int hs = hact ? h : 0;
    const int hk = hs % p.Hk;

    // ---- query weights of this thread's 8 dims (scale and log2(e) folded in) -----
    // rotated dims: (wa, wb) as an fp16 pair for v_dot2 with the (cos, sin) table pair
    float wa[8], wb[8];
    f16x2 wab[8];
    {
      const float2* qwr = p.qw + ((int64_t)b * p.Hq + hs) * D + min(d0, D - 8);
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float2 w = cact ? qwr[s] : make_float2(0.f, 0.f);
        wa[s] = w.x;
        wb[s] = w.y;
        wab[s] = f16x2{(_Float16)wa[s], (_Float16)wb[s]};
      }
    }
    const uint16_t* kbase = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1];
    const uint16_t* vbase = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];

    // ---- pass 1: scaled scores into LDS ---------------------------------------------
    // two register sets alternate (no copies): while one batch is computed, the next
    // one's loads are in flight
    u32x4 bufA[kBatch], bufB[kBatch];
    // Branch-free loads, so the compiler can count them and wait only for the batch it computes:
    // every lane reads a valid address (rows past the cache clamp to its last row, chunks past D
    // to the last chunk, idle lanes read their head's rows; their data meet zero weights or are
    // never stored).  Masked keys are dropped at the score, so no load waits on a mask byte.
    // Offsets within one (batch, head) fit in 32 bits (checked on the host).
    // per lane: its first row (key j_begin + kp; idle lanes take the last parity) and how many
    // rows past it exist, so a load needs one clamp and one multiply-add
    const int kpl = min(kp, KP - 1);
    const int rows_left = Nk - 1 - j_begin - kpl;
    const int ks2 = (int)p.k_s[2], vs2 = (int)p.v_s[2];
    const uint16_t* klane = kbase + ((j_begin + kpl) * ks2 + min(d0, D - 8));
    const uint16_t* vlane = vbase + ((j_begin + kpl) * vs2 + min(d0, D - 8));
    auto fetch = [&](u32x4* buf, const uint16_t* lanep, int row_stride, int bt) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int r = min((bt * kBatch + u) * KP, rows_left);
        buf[u] = ld16(lanep + r * row_stride);
      }
    };
    // LDS byte address of the lane's table chunk in row 0 (lanes past D read the last staged
    // chunk: finite values that meet their zero weights)
    const uint32_t tab_lane = lds_addr(tab_s + min(d0, max(R, 8) - 8));
    // every dim rotated (R == D): one straight-line score per key, softplus(x) = max(x, 0) +
    // ln 2 log2(1 + 2^(-|x| log2 e)) with the max taken on the bit pattern (x >= 0 iff its
    // signed bits are), no per-key branch
    auto score_rot = [&](const u32x4* cur, int bt) {
      // the batch's keys side by side: independent chains between the transcendentals and the
      // dot products (no dependent back-to-back instructions)
      float part[kBatch];
      u32x4 t0[kBatch], t1[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int jl = kp + (bt * kBatch + u) * KP;
        const uint32_t ta = tab_lane + 4 * TS * min(jl, kSplit - 1);
        t0[u] = lds_read16_at(ta);
        t1[u] = lds_read16_at(ta + 16);
        part[u] = 0.f;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        float e[kBatch], mx[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const uint32_t w = cur[u][q >> 1];
          const uint32_t xb = T::kCode == 2 ? ((q & 1) ? (w & 0xffff0000u) : (w << 16))
                                            : __builtin_bit_cast(uint32_t, T::to_float((uint16_t)((q & 1) ? (w >> 16) : (w & 0xffffu))));
          e[u] = __builtin_amdgcn_exp2f(-fabsf(__builtin_bit_cast(float, xb)) * kLog2e);
          mx[u] = __builtin_bit_cast(float, max((int)xb, 0));
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) e[u] = __builtin_amdgcn_logf(1.f + e[u]);
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const f16x2 cs = __builtin_bit_cast(f16x2, q < 4 ? t0[u][q] : t1[u][q - 4]);
          part[u] = fmaf(fmaf(e[u], kLn2, mx[u]), __builtin_amdgcn_fdot2(cs, wab[q], 0.f, false), part[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int jl = kp + (bt * kBatch + u) * KP;
        const float sc = group_sum<LPK>(part[u]);
        if (c == 0 && active && jl < kSplit) s_lds[hl][jl] = vis_s[jl] ? sc : -INFINITY;
      }
    };
    auto score = [&](const u32x4* cur, int bt) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int jl = kp + (bt * kBatch + u) * KP;
        float x[8];
        unpack8<T>(cur[u], x);
        float part = 0.f;
        if (rot) {
          const u32x4* t = reinterpret_cast<const u32x4*>(tab_s + min(jl, kSplit - 1) * TS + d0);
          const u32x4 t0 = t[0], t1 = t[1];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            // (cos, sin) of dim d0 + q dotted with (wa, wb), accumulated in fp32
            const f16x2 cs = __builtin_bit_cast(f16x2, q < 4 ? t0[q] : t1[q - 4]);
            part = fmaf(softplus_f(x[q]), __builtin_amdgcn_fdot2(cs, wab[q], 0.f, false), part);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q) part += wa[q] * x[q];
        }
        part = group_sum<LPK>(part);
        if (c == 0 && active && jl < kSplit) s_lds[hl][jl] = vis_s[jl] ? part : -INFINITY;
      }
    };
    // straight-line prefetch (the last pair peeled): while one batch is computed the next is in
    // flight, and the first V batch is in flight while the K pass ends and the maxima are reduced
    auto kpass = [&](auto all_rot) {
      auto sc = [&](const u32x4* cur, int bt) {
        if constexpr (decltype(all_rot)::value) score_rot(cur, bt);
        else score(cur, bt);
      };
      fetch(bufA, klane, ks2, 0);
      for (int bt = 0; bt + 2 < nbu; bt += 2) {
        fetch(bufB, klane, ks2, bt + 1);
        sc(bufA, bt);
        fetch(bufA, klane, ks2, bt + 2);
        sc(bufB, bt + 1);
      }
      fetch(bufB, klane, ks2, nbu - 1);
      sc(bufA, nbu - 2);
      fetch(bufA, vlane, vs2, 0);
      sc(bufB, nbu - 1);
    };
    if (R == D) kpass(std::true_type{});
    else kpass(std::false_type{});
    __syncthreads();

    // ---- each head's max over the split (LPK * KP threads per head) -----------------
    float mx = -INFINITY;
    if (hact)
      for (int i = c + LPK * kp; i < kSplit; i += LPK * KP) mx = fmaxf(mx, s_lds[hl][i]);
    red_o[tid][0] = mx;   // partial max per (hl, kp, c)
    __syncthreads();
    if (hact) {
      float m2 = -INFINITY;
      for (int k2 = 0; k2 < KP; ++k2)
        for (int c2 = 0; c2 < LPK; ++c2) m2 = fmaxf(m2, red_o[(hl + HG * k2) * LPK + c2][0]);
      mx = m2;
    }
    __syncthreads();
    const float mu = mx == -INFINITY ? 0.f : mx;

    // ---- pass 2: p = exp2(s - m), o += p v ---------------------------------------
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float lsum = 0.f;
    auto accumulate = [&](const u32x4* cur, int bt) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int jl = kp + (bt * kBatch + u) * KP;
        const float pv = jl < kSplit ? __builtin_amdgcn_exp2f(s_lds[hl][jl] - mu) : 0.f;   // 0 when masked
        float x[8];
        unpack8<T>(cur[u], x);
#pragma unroll
        for (int s = 0; s < 8; ++s) acc[s] = fmaf(pv, x[s], acc[s]);
        lsum += pv;
      }
    };
    for (int bt = 0; bt + 2 < nbu; bt += 2) {
      fetch(bufB, vlane, vs2, bt + 1);
      accumulate(bufA, bt);
      fetch(bufA, vlane, vs2, bt + 2);
      accumulate(bufB, bt + 1);
    }
    fetch(bufB, vlane, vs2, nbu - 1);
    accumulate(bufA, nbu - 2);
    accumulate(bufB, nbu - 1);

    // ---- merge the KP key parities of each (head, chunk), write the partial -------
#pragma unroll
    for (int s = 0; s < 8; ++s) red_o[tid][s] = acc[s];
    if (c == 0) red_ml[rest][1] = lsum;
    __syncthreads();
    if (hact && kp == 0) {
      float o8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      float L = 0.f;
      for (int k2 = 0; k2 < KP; ++k2) {
        const int r2 = hl + HG * k2;
        L += red_ml[r2][1];
#pragma unroll
        for (int s = 0; s < 8; ++s) o8[s] += red_o[r2 * LPK + c][s];
      }
      const int64_t row = ((int64_t)b * p.Hq + h) * p.splits + split;
      if (cact) {
#pragma unroll
        for (int s = 0; s < 8; ++s)
          if (d0 + s < D) p.part_o[row * D + d0 + s] = o8[s];
      }
      if (c == 0) {
        p.part_ml[row * 2] = mx;
        p.part_ml[row * 2 + 1] = L;
      }
    }
    __syncthreads();
  }
}

// One workgroup per (batch, head): merge the splits by log-sum-exp.
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams p) {
  __shared__ float w_s[1024];
  __shared__ float red[4];
  __shared__ float part[4][128];
  const int bh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = bh / p.Hq, h = bh % p.Hq;
  const int D = p.D, S = p.splits;
  const float* pml = p.part_ml + (int64_t)bh * S * 2;
  const float* po = p.part_o + (int64_t)bh * S * D;
  float M = -INFINITY;
  for (int s = tid; s < S; s += 256) M = fmaxf(M, pml[2 * s]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) M = fmaxf(M, __shfl_xor(M, m, 64));
  if (lane == 0) red[wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float Mu = M == -INFINITY ? 0.f : M;
  __syncthreads();
  float L = 0.f;
  for (int s = tid; s < S; s += 256) {
    const float w = __builtin_amdgcn_exp2f(pml[2 * s] - Mu);
    if (s < 1024) w_s[s] = w;
    L += pml[2 * s + 1] * w;
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) L += __shfl_xor(L, m, 64);
  if (lane == 0) red[wave] = L;
  __syncthreads();
  L = red[0] + red[1] + red[2] + red[3];
  const float inv = L > 0.f ? 1.f / L : 0.f;
  // thread = (split group g of 4, dim d): 4 groups x up to 64 dims per pass
  for (int d0 = 0; d0 < D; d0 += 64) {
    const int d = d0 + lane;
    float acc = 0.f;
    if (d < D) {
      int s = wave;
      for (; s + 28 < S; s += 32) {   // 8 independent loads in flight
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = po[(int64_t)(s + 4 * u) * D + d];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int su = s + 4 * u;
          acc += v[u] * (su < 1024 ? w_s[su] : __builtin_amdgcn_exp2f(pml[2 * su] - Mu));
        }
      }
      for (; s < S; s += 4) acc += po[(int64_t)s * D + d] * (s < 1024 ? w_s[s] : __builtin_amdgcn_exp2f(pml[2 * s] - Mu));
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && d < D) {
      uint16_t* orow = p.o + (int64_t)b * p.o_s[0] + (int64_t)h * p.o_s[1];
      orow[d] = T::bits((part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane]) * inv);
    }
    __syncthreads();
  }
  if (tid == 0) p.lse[bh] = L > 0.f ? (M + __builtin_amdgcn_logf(L)) * kLn2 : -INFINITY;
}

template <typename T, int LPK, int RMAX>
hipError_t launch_t(const DecodeParams& p, hipStream_t s) {
  int HG = kThreads / LPK < kMaxHG ? kThreads / LPK : kMaxHG;
  if (p.Hq < HG) HG = p.Hq;
  const int KP = (kThreads / LPK) / HG;
  const int64_t n_tab = p.R > 0 ? (int64_t)(p.t_sb != 0 ? p.B : 1) * p.Nk * p.R : 0;
  const int tab_blocks = (int)((n_tab + 1023) / 1024);   // 4 entries per thread
  const int qw_blocks = (p.B * p.Hq * p.D + 255) / 256;
  hipError_t e = launch_named("flash_decode_setup", decode_setup_kernel<T>, dim3(tab_blocks + qw_blocks), dim3(256),
                              s, p, tab_blocks, n_tab);
  if (e != hipSuccess) return e;
  e = launch_named("flash_decode_split", decode_split_kernel<T, LPK, RMAX>, dim3(p.B * p.splits),
                   dim3(kThreads), s, p, HG, KP);
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

int decode_split_keys() { return kSplit; }

hipError_t launch_flash_decode(const DecodeParams& p, int dtype, hipStream_t s) {
  // per-head phase tables would need a table chunk per head: the general forward covers them
  if (p.Nq != 1 || p.causal || p.D > 128 || p.t_sh != 0) return hipErrorInvalidValue;
  return dtype == 2 ? dispatch<BF16>(p, s) : dispatch<F16>(p, s);
}

}  // namespace pope
