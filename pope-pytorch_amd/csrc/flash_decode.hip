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
//   decode_split : one workgroup (4 waves) per (batch, query head, split of
//                  kSplit keys).  A split whose keys are all masked exits after
//                  reading its mask bytes.  Pass 1 streams K: LPK lanes share one
//                  key row (16 bytes each, coalesced), apply the polar transform
//                  of the key -- softplus(k) times cos / sin of the key phase from
//                  the per-call table -- fold in the query's (cos, sin) weights
//                  and reduce the score across the LPK lanes; the scaled scores
//                  of the split go to LDS.  Pass 2 takes the split's max, streams
//                  V with the same lane mapping and accumulates p * v; the
//                  partial (m, l, o) is written to the workspace.
//   decode_combine : merges the splits of each (batch, head) by their log-sum-exp
//                  and writes o (input dtype) and lse (natural log, -inf when
//                  every key is masked).
// The query weights use the bias-on-the-query-side form of the score,
//   a_d c_jd cos((F_q,d - b_d) - F_j,d)
//     = c_jd [a_d cos(F_q,d - b_d) cos F_j,d + a_d sin(F_q,d - b_d) sin F_j,d],
// so the key side needs only cos / sin(F_j) (shared by every head and batch).
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kThreads = 256;
constexpr int kSplit = 512;    // keys per split (one workgroup)
constexpr int kUnroll = 4;     // key steps whose loads are issued together

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

template <typename T, int LPK>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeParams p) {
  constexpr int KPW = 64 / LPK;                // keys per wave step
  constexpr int KPS = 4 * KPW;                 // keys per workgroup step
  constexpr int NSTEP = kSplit / KPS;
  __shared__ float s_lds[kSplit];
  __shared__ float red[4][128];
  __shared__ float red_l[4];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int split = blockIdx.x % p.splits;
  const int bh = blockIdx.x / p.splits;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int D = p.D, R = p.R, Nk = p.Nk;
  const int ks = lane / LPK, c = lane % LPK, d0 = 8 * c;
  const bool cact = d0 < D;
  const int j_begin = split * kSplit;
  const uint8_t* mrow = p.has_mask ? p.mask + (int64_t)b * p.mask_sb : nullptr;
  float* po = p.part_o + ((int64_t)bh * p.splits + split) * D;
  float* pml = p.part_ml + ((int64_t)bh * p.splits + split) * 2;

  // ---- skip splits without a visible key ----------------------------------
  int vis_any = 0;
  for (int j = j_begin + tid; j < min(j_begin + kSplit, Nk); j += kThreads)
    vis_any |= (!p.has_mask || mrow[j] != 0);
  if (!__syncthreads_or(vis_any)) {
    if (tid < D) po[tid] = 0.f;
    if (tid == 0) {
      pml[0] = -INFINITY;
      pml[1] = 0.f;
    }
    return;
  }

  // ---- query weights of this lane's 8 dims ----------------------------------
  float wa[8], wb[8];
  {
    const int q_off = Nk - 1;
    const uint16_t* qrow = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1];
    float x[8];
    unpack8<T>(cact ? ld16(qrow + d0) : u32x4{0u, 0u, 0u, 0u}, x);
    const float* frow = R ? p.freqs + (int64_t)b * p.f_s[0] + (int64_t)h * p.f_s[1] + (int64_t)q_off * p.f_s[2] : nullptr;
    const float* brow = R ? p.bias + (int64_t)hk * p.bias_sh : nullptr;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int d = d0 + s;
      if (cact && d < R) {
        float sn, cs;
        sincos_acc(frow[d] - brow[d], &sn, &cs);
        const float a = softplus_f(x[s]);
        wa[s] = a * cs;
        wb[s] = a * sn;
      } else {
        wa[s] = cact ? x[s] : 0.f;
        wb[s] = 0.f;
      }
    }
  }

  const uint16_t* kbase = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1];
  const uint16_t* vbase = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  const float2* tbase = R ? p.table + (int64_t)b * p.t_sb + (int64_t)h * p.t_sh : nullptr;
  const bool rot = cact && d0 < R;   // R is a multiple of 8: a chunk is all rotated or all pass-through

  // ---- pass 1: scaled scores of the split's keys into LDS ---------------------
  for (int st0 = 0; st0 < NSTEP; st0 += kUnroll) {
    u32x4 kr[kUnroll];
    float4 tc[kUnroll][4];
    bool ok[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int j = j_begin + (st0 + u) * KPS + wave * KPW + ks;
      ok[u] = j < Nk && (!p.has_mask || mrow[j] != 0);
      const int jj = min(j, Nk - 1);
      kr[u] = (ok[u] && cact) ? ld16(kbase + (int64_t)jj * p.k_s[2] + d0) : u32x4{0u, 0u, 0u, 0u};
      if (rot) {
        const float4* t = reinterpret_cast<const float4*>(tbase + (int64_t)jj * R + d0);
#pragma unroll
        for (int q = 0; q < 4; ++q) tc[u][q] = t[q];
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float x[8];
      unpack8<T>(kr[u], x);
      float part = 0.f;
      if (rot) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 t = tc[u][q];   // (cos, sin) of dims d0 + 2q, d0 + 2q + 1
          part += softplus_f(x[2 * q]) * (wa[2 * q] * t.x + wb[2 * q] * t.y);
          part += softplus_f(x[2 * q + 1]) * (wa[2 * q + 1] * t.z + wb[2 * q + 1] * t.w);
        }
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) part += wa[s] * x[s];
      }
#pragma unroll
      for (int m = 1; m < LPK; m <<= 1) part += __shfl_xor(part, m, 64);
      if (c == 0) {
        const int jl = (st0 + u) * KPS + wave * KPW + ks;
        s_lds[jl] = ok[u] ? part * p.scale_log2 : -INFINITY;
      }
    }
  }
  __syncthreads();

  // ---- split max ---------------------------------------------------------------
  float mx = -INFINITY;
  for (int i = tid; i < kSplit; i += kThreads) mx = fmaxf(mx, s_lds[i]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
  if (lane == 0) red[wave][0] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[1][0]), fmaxf(red[2][0], red[3][0]));
  __syncthreads();

  // ---- pass 2: p = exp2(s - m), o += p v ---------------------------------------
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
  for (int st0 = 0; st0 < NSTEP; st0 += kUnroll) {
    u32x4 vr[kUnroll];
    float pv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int jl = (st0 + u) * KPS + wave * KPW + ks;
      const int j = j_begin + jl;
      pv[u] = __builtin_amdgcn_exp2f(s_lds[jl] - mx);   // 0 for masked keys (s = -inf)
      vr[u] = (pv[u] > 0.f && cact) ? ld16(vbase + (int64_t)min(j, Nk - 1) * p.v_s[2] + d0) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float x[8];
      unpack8<T>(vr[u], x);
#pragma unroll
      for (int s = 0; s < 8; ++s) acc[s] = fmaf(pv[u], x[s], acc[s]);
      lsum += pv[u];
    }
  }
  // reduce over the key slots of the wave (lanes with the same chunk), then over waves
#pragma unroll
  for (int m = LPK; m < 64; m <<= 1) {
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[s] += __shfl_xor(acc[s], m, 64);
    lsum += __shfl_xor(lsum, m, 64);
  }
  if (ks == 0) {
#pragma unroll
    for (int s = 0; s < 8; ++s) red[wave][d0 + s] = acc[s];
    if (c == 0) red_l[wave] = lsum;
  }
  __syncthreads();
  if (tid < D) po[tid] = red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid];
  if (tid == 0) {
    pml[0] = mx;
    pml[1] = red_l[0] + red_l[1] + red_l[2] + red_l[3];
  }
}

// One wave per (batch, head): merge the splits by log-sum-exp.
template <typename T>
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeParams p) {
  const int bh = blockIdx.x, lane = threadIdx.x;
  const int b = bh / p.Hq, h = bh % p.Hq;
  const int D = p.D, S = p.splits;
  const float* pml = p.part_ml + (int64_t)bh * S * 2;
  const float* po = p.part_o + (int64_t)bh * S * D;
  float M = -INFINITY;
  for (int s = lane; s < S; s += 64) M = fmaxf(M, pml[2 * s]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) M = fmaxf(M, __shfl_xor(M, m, 64));
  const float Mu = M == -INFINITY ? 0.f : M;
  float L = 0.f;
  for (int s = lane; s < S; s += 64) L += pml[2 * s + 1] * __builtin_amdgcn_exp2f(pml[2 * s] - Mu);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) L += __shfl_xor(L, m, 64);
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t* orow = p.o + (int64_t)b * p.o_s[0] + (int64_t)h * p.o_s[1];
  for (int d = lane; d < D; d += 64) {
    float acc = 0.f;
    for (int s = 0; s < S; ++s) acc += po[(int64_t)s * D + d] * __builtin_amdgcn_exp2f(pml[2 * s] - Mu);
    orow[d] = T::bits(acc * inv);
  }
  if (lane == 0) p.lse[bh] = L > 0.f ? (M + __builtin_amdgcn_logf(L)) * kLn2 : -INFINITY;
}

template <typename T, int LPK>
hipError_t launch_t(const DecodeParams& p, hipStream_t s) {
  hipError_t e = launch_named("flash_decode_split", decode_split_kernel<T, LPK>, dim3(p.B * p.Hq * p.splits),
                              dim3(kThreads), s, p);
  if (e != hipSuccess) return e;
  return launch_named("flash_decode_combine", decode_combine_kernel<T>, dim3(p.B * p.Hq), dim3(64), s, p);
}

template <typename T>
hipError_t dispatch(const DecodeParams& p, hipStream_t s) {
  const int chunks = p.D / 8;
  if (chunks <= 4) return launch_t<T, 4>(p, s);
  if (chunks <= 8) return launch_t<T, 8>(p, s);
  if (chunks <= 16) return launch_t<T, 16>(p, s);
  return hipErrorInvalidValue;
}

}  // namespace

int decode_split_keys() { return kSplit; }

hipError_t launch_flash_decode(const DecodeParams& p, int dtype, hipStream_t s) {
  if (p.Nq != 1 || p.causal || p.D > 128) return hipErrorInvalidValue;
  return dtype == 2 ? dispatch<BF16>(p, s) : dispatch<F16>(p, s);
}

}  // namespace pope
