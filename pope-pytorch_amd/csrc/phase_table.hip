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
  const int64_t total = (int64_t)p.Bt * p.Ht * p.rows * p.R;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int d = (int)(idx % p.R);
    int64_t rest = idx / p.R;
    const int n = (int)(rest % p.rows);
    rest /= p.rows;
    const int ht = (int)(rest % p.Ht);
    const int bt = (int)(rest / p.Ht);
    float th = p.freqs[(int64_t)bt * p.f_sb + (int64_t)ht * p.f_sh + (int64_t)n * p.f_sn + d];
    if (p.bias) th = th + p.bias[(int64_t)ht * p.bias_sh + d];
    float s, c;
    sincos_acc(th, &s, &c);
    if (p.out16) {
      const f16x2 v = {(_Float16)c, (_Float16)s};
      p.out16[idx] = __builtin_bit_cast(uint32_t, v);
    } else {
      p.out[idx] = make_float2(c, s);
    }
  }
}

hipError_t launch_phase_table(const TableParams& p, hipStream_t s) {
  const int64_t total = (int64_t)p.Bt * p.Ht * p.rows * p.R;
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  return launch_named("phase_table", phase_table_kernel, dim3((unsigned)blocks), dim3(256), s, p);
}

}  // namespace pope
