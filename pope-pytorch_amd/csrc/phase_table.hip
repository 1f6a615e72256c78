// Per-call cos/sin table of the PoPE phases.
//
// tab[((bt * Ht + ht) * rows + n) * R + d] = (cos th, sin th), fp32 pairs or fp16 pairs,
//   th = fl(F[bt, ht, n, d] + bias[ht, d])   (bias optional)
// The sum is rounded to fp32 before the trig call, as the reference does
// (freqs_with_bias = freqs + bias, pope.py:56; theta_k = fk + bias,
// triton_pope.py:76).  The table depends on positions only (not on q/k data),
// so it is shared by every (batch, head) that reads the same phases.
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

__global__ __launch_bounds__(256) void phase_table_kernel(TableParams p) {
  // four consecutive entries of one row per thread (R is a multiple of 8): four independent
  // loads, 16-byte stores; the index is decomposed in 32 bits when the table allows
  const int64_t total = (int64_t)p.Bt * p.Ht * p.rows * p.R;
  for (int64_t i4 = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x); i4 < total; i4 += 4 * (int64_t)gridDim.x * 256) {
    int d, n, ht, bt;
    if (total < INT32_MAX) {
      const int i = (int)i4;
      d = i % p.R;
      int rest = i / p.R;
      n = rest % p.rows;
      rest /= p.rows;
      ht = rest % p.Ht;
      bt = rest / p.Ht;
    } else {
      d = (int)(i4 % p.R);
      int64_t rest = i4 / p.R;
      n = (int)(rest % p.rows);
      rest /= p.rows;
      ht = (int)(rest % p.Ht);
      bt = (int)(rest / p.Ht);
    }
    const float* f = p.freqs + (int64_t)bt * p.f_sb + (int64_t)ht * p.f_sh + (int64_t)n * p.f_sn + d;
    float th[4], sn[4], cs[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) th[t] = f[t];
    if (p.bias) {
      const float* bb = p.bias + (int64_t)ht * p.bias_sh + d;
#pragma unroll
      for (int t = 0; t < 4; ++t) th[t] = th[t] + bb[t];
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) sincos_acc(th[t], &sn[t], &cs[t]);
    if (p.out16) {
      u32x4 w;
#pragma unroll
      for (int t = 0; t < 4; ++t) w[t] = __builtin_bit_cast(uint32_t, f16x2{(_Float16)cs[t], (_Float16)sn[t]});
      *reinterpret_cast<u32x4*>(p.out16 + i4) = w;
    } else {
      float4* dst = reinterpret_cast<float4*>(p.out + i4);
      dst[0] = make_float4(cs[0], sn[0], cs[1], sn[1]);
      dst[1] = make_float4(cs[2], sn[2], cs[3], sn[3]);
    }
  }
}

hipError_t launch_phase_table(const TableParams& p, hipStream_t s) {
  const int64_t total = (int64_t)p.Bt * p.Ht * p.rows * p.R;
  if (total == 0) return hipSuccess;
  int64_t blocks = (total / 4 + 255) / 256;   // four entries per thread
  if (blocks > 4096) blocks = 4096;
  return launch_named("phase_table", phase_table_kernel, dim3((unsigned)blocks), dim3(256), s, p);
}

}  // namespace pope
