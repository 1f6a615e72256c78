// Phase (cos, sin) of one rotated dim of the similarity, computed where a kernel needs it instead
// of read from a precomputed table:
//   side 0, query row of head h:    theta = F[b, h, n, d]                  (n = Nk - Nq + i, no bias)
//   side 1, key row of kv head hk:  theta = fl(F[b, hk, n, d] + bias[hk, d])   (pope.py:56,
//                                   triton_pope.py:76: the sum is rounded to fp32 first)
// freqs and bias broadcast over batch / head through zero strides.  sincos_rev: FMA-split
// reduction to revolutions and the hardware sine / cosine, max abs error 2e-7 for |theta| <= 1e6.
#pragma once

#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

__device__ __forceinline__ float2 sim_phase(const SimParams& p, int side, int b, int hh, int n, int d) {
  float th = p.freqs[(int64_t)b * p.f_s[0] + (int64_t)hh * p.f_s[1] + (int64_t)n * p.f_s[2] + d];
  if (side == 1) th = th + p.bias[(int64_t)hh * p.bias_sh + d];
  float s, c;
  sincos_rev(th, &s, &c);
  return make_float2(c, s);
}

}  // namespace pope
