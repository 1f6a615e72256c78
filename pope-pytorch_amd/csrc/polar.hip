// Materialising PoPE polar transform on the device (gfx950): apply_pope_to_qk
// (pope.py:30-86) forward and backward.
//
//   q_hat[..., 2d]     = a_d cos(phi_d),  q_hat[..., 2d + 1] = a_d sin(phi_d)      d < R
//   q_hat[..., R + d]  = q_d                                                      d >= R
// with a = softplus(q) rounded to q's dtype (the reference applies F.softplus to the input
// tensor, pope.py:60, then multiplies by fp32 cos / sin, which promotes, :69-70), the query
// phase phi = F[q_off + i] (right-aligned rows, :64) and the key phase psi = fl(F[j] + bias[h])
// (the bias added in fp32 before cos / sin, :56).  Outputs are fp32 (B, H, N, D + R) rows.
//
// Backward, per rotated dim (g = the output gradient):
//   dq   = sigmoid(q) (cos phi g_2d + sin phi g_2d+1)          (in q's dtype)
//   dphi = a (cos phi g_2d+1 - sin phi g_2d)                    -> dfreqs rows, dbias (keys)
// Pass-through dims copy g.  dfreqs and dbias are fp32 and accumulated (atomics; dbias summed
// over the workgroup's rows first).
//
// Complex layout (return_complex, pope.py:49-51,66-67,74-75): rows of D (re, im) fp32 pairs, the
// memory layout of torch.polar's complex64 output.  The rotated dims are the same interleaved
// pairs; pass-through dim d is the pair (q_d, 0) at columns 2d, 2d + 1, and its gradient is
// sign(q_d) times the real part of the pair's gradient (torch.polar's backward for a possibly
// negative magnitude, which the reference's torch path differentiates).
//
// One thread per (row, 4 input dims); a workgroup covers 256 / (D / 4) rows of one (batch, head)
// (grid y), so the dbias partial sums reduce in LDS.
#include <type_traits>

#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kThreads = 256;

template <typename T>
__device__ __forceinline__ void load4(const void* base, int64_t off, float* x) {
  if constexpr (std::is_same<T, float>::value) {
    const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  } else {
    const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(base) + off);
    x[0] = T::to_float((uint16_t)(w[0] & 0xffffu));
    x[1] = T::to_float((uint16_t)(w[0] >> 16));
    x[2] = T::to_float((uint16_t)(w[1] & 0xffffu));
    x[3] = T::to_float((uint16_t)(w[1] >> 16));
  }
}

template <typename T>
__device__ __forceinline__ void store4(void* base, int64_t off, const float* x) {
  if constexpr (std::is_same<T, float>::value) {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + off) = make_float4(x[0], x[1], x[2], x[3]);
  } else {
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(base) + off) = u32x2{T::pack2(x[0], x[1]), T::pack2(x[2], x[3])};
  }
}

// Rounds to T's precision (identity for fp32).
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (std::is_same<T, float>::value) return v;
  else return T::to_float(T::bits(v));
}

struct Side {
  const void* x; int64_t xs0, xs1, xs2;   // q or k
  float* out;                             // (heads, N, D + R) fp32
  const float* gout;                      // its gradient (backward)
  void* dx; int64_t ds0, ds1, ds2;        // dq or dk (backward)
  int H, N, frow0, key;                   // heads, rows, first phase row, 1 = key side (bias)
};

// phases of the thread's 4 rotated dims
__device__ __forceinline__ void phases(const PolarParams& p, const Side& sd, int b, int h, int n, int d0, float* ph,
                                       int& frow) {
  frow = sd.frow0 + n;
  const float* f = p.freqs + (int64_t)b * p.f_s[0] + (int64_t)h * p.f_s[1] + (int64_t)frow * p.f_s[2] + d0;
#pragma unroll
  for (int t = 0; t < 4; ++t) ph[t] = f[t];
  if (sd.key) {
    const float* bb = p.bias + (int64_t)h * p.bias_sh + d0;
#pragma unroll
    for (int t = 0; t < 4; ++t) ph[t] = ph[t] + bb[t];
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void polar_fwd_kernel(PolarParams p, Side sd) {
  const int U = p.D / 4, rpb = kThreads / U;
  const int u = threadIdx.x % U, r = threadIdx.x / U;
  const int bh = blockIdx.y, n = blockIdx.x * rpb + r;
  if (r >= rpb || n >= sd.N) return;
  const int b = bh / sd.H, h = bh % sd.H;
  const int d0 = 4 * u, E = p.cplx ? 2 * p.D : p.D + p.R;
  float x[4];
  load4<T>(sd.x, (int64_t)b * sd.xs0 + (int64_t)h * sd.xs1 + (int64_t)n * sd.xs2 + d0, x);
  float* orow = sd.out + ((int64_t)bh * sd.N + n) * E;
  if (d0 < p.R) {
    float ph[4];
    int frow;
    phases(p, sd, b, h, n, d0, ph, frow);
    float o[8];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float sn, cs;
      sincos_acc(ph[t], &sn, &cs);
      const float a = round_to<T>(softplus_f(x[t]));
      o[2 * t] = a * cs;
      o[2 * t + 1] = a * sn;
    }
    *reinterpret_cast<float4*>(orow + 2 * d0) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4*>(orow + 2 * d0 + 4) = make_float4(o[4], o[5], o[6], o[7]);
  } else if (p.cplx) {
    *reinterpret_cast<float4*>(orow + 2 * d0) = make_float4(x[0], 0.f, x[1], 0.f);
    *reinterpret_cast<float4*>(orow + 2 * d0 + 4) = make_float4(x[2], 0.f, x[3], 0.f);
  } else {
    *reinterpret_cast<float4*>(orow + p.R + d0) = make_float4(x[0], x[1], x[2], x[3]);
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void polar_bwd_kernel(PolarParams p, Side sd) {
  __shared__ float red[kThreads][4];
  const int U = p.D / 4, rpb = kThreads / U;
  const int u = threadIdx.x % U, r = threadIdx.x / U;
  const int bh = blockIdx.y, n = blockIdx.x * rpb + r;
  const bool live = r < rpb && n < sd.N;
  const int b = bh / sd.H, h = bh % sd.H;
  const int d0 = 4 * u, E = p.cplx ? 2 * p.D : p.D + p.R;
  float dph[4] = {0.f, 0.f, 0.f, 0.f};
  if (live) {
    float x[4];
    load4<T>(sd.x, (int64_t)b * sd.xs0 + (int64_t)h * sd.xs1 + (int64_t)n * sd.xs2 + d0, x);
    const float* grow = sd.gout + ((int64_t)bh * sd.N + n) * E;
    const int64_t doff = (int64_t)b * sd.ds0 + (int64_t)h * sd.ds1 + (int64_t)n * sd.ds2 + d0;
    float dx[4];
    if (d0 < p.R) {
      float ph[4];
      int frow;
      phases(p, sd, b, h, n, d0, ph, frow);
      const float4 g0 = *reinterpret_cast<const float4*>(grow + 2 * d0);
      const float4 g1 = *reinterpret_cast<const float4*>(grow + 2 * d0 + 4);
      const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float sn, cs;
        sincos_acc(ph[t], &sn, &cs);
        const float a = round_to<T>(softplus_f(x[t]));
        dx[t] = sigmoid_f(x[t]) * (cs * g[2 * t] + sn * g[2 * t + 1]);
        dph[t] = a * (cs * g[2 * t + 1] - sn * g[2 * t]);
      }
      float* part = sd.key ? p.kpart : p.qpart;   // deterministic mode: written once, summed later
      if (part) {
        float* dst = part + (((int64_t)b * sd.H + h) * sd.N + n) * p.R + d0;
#pragma unroll
        for (int t = 0; t < 4; ++t) dst[t] = dph[t];
      } else if (p.dfreqs) {
        float* df = p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)h * p.df_s[1] + (int64_t)frow * p.df_s[2] + d0;
#pragma unroll
        for (int t = 0; t < 4; ++t) atomicAdd(df + t, dph[t]);
      }
    } else if (p.cplx) {
      // real parts of the (re, im) gradient pairs, times sign(x): the reference builds the pair
      // with torch.polar(x, 0) (pope.py:50-51), whose backward takes Re(g * conj(sgn(result)))
      const float4 g0 = *reinterpret_cast<const float4*>(grow + 2 * d0);
      const float4 g1 = *reinterpret_cast<const float4*>(grow + 2 * d0 + 4);
      const float gr[4] = {g0.x, g0.z, g1.x, g1.z};
#pragma unroll
      for (int t = 0; t < 4; ++t) dx[t] = x[t] > 0.f ? gr[t] : x[t] < 0.f ? -gr[t] : 0.f;
    } else {
      const float4 g = *reinterpret_cast<const float4*>(grow + p.R + d0);
      dx[0] = g.x; dx[1] = g.y; dx[2] = g.z; dx[3] = g.w;
    }
    store4<T>(sd.dx, doff, dx);
  }
  if (sd.key && p.dbias && !p.kpart) {   // sum the workgroup's rows per dim, one atomic per dim
#pragma unroll
    for (int t = 0; t < 4; ++t) red[threadIdx.x][t] = dph[t];
    __syncthreads();
    if (r == 0 && d0 < p.R) {
      float s4[4] = {0.f, 0.f, 0.f, 0.f};
      for (int r2 = 0; r2 < rpb; ++r2)
#pragma unroll
        for (int t = 0; t < 4; ++t) s4[t] += red[r2 * U + u][t];
      float* db = p.dbias + (int64_t)h * p.bias_sh + d0;
#pragma unroll
      for (int t = 0; t < 4; ++t) atomicAdd(db + t, s4[t]);
    }
  }
}

template <typename T>
hipError_t launch_side(const PolarParams& p, const Side& sd, bool bwd, hipStream_t s) {
  const int U = p.D / 4, rpb = kThreads / U;
  const dim3 grid((unsigned)((sd.N + rpb - 1) / rpb), (unsigned)(p.B * sd.H));
  if (bwd) return launch_named("polar_bwd", polar_bwd_kernel<T>, grid, dim3(kThreads), s, p, sd);
  return launch_named("polar_fwd", polar_fwd_kernel<T>, grid, dim3(kThreads), s, p, sd);
}

template <typename T>
hipError_t launch_t(const PolarParams& p, bool bwd, hipStream_t s) {
  Side q{p.q, p.q_s[0], p.q_s[1], p.q_s[2], p.qh, p.gq, p.dq, p.dq_s[0], p.dq_s[1], p.dq_s[2],
         p.Hq, p.Nq, p.Nk - p.Nq, 0};
  Side k{p.k, p.k_s[0], p.k_s[1], p.k_s[2], p.kh, p.gk, p.dk, p.dk_s[0], p.dk_s[1], p.dk_s[2],
         p.Hk, p.Nk, 0, 1};
  hipError_t e = launch_side<T>(p, q, bwd, s);
  if (e != hipSuccess) return e;
  return launch_side<T>(p, k, bwd, s);
}

}  // namespace

hipError_t launch_polar(const PolarParams& p, int dtype, bool bwd, hipStream_t s) {
  if (dtype == 0) return launch_t<float>(p, bwd, s);
  if (dtype == 1) return launch_t<F16>(p, bwd, s);
  return launch_t<BF16>(p, bwd, s);
}

}  // namespace pope
