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

// Clears the phase gradients the finalize accumulates into, over what the backward addresses:
// dfreqs rows n < Nk of every (bt, ht) and the Hb rows of dbias.  Called by every thread of the
// backward's first launch with its flat index and the launch's thread count.
__device__ __forceinline__ void sim_clear_grads(const SimParams& p, int64_t gid, int64_t nthreads) {
  const int R = p.R;
  if (p.dbias)
    for (int64_t x = gid; x < (int64_t)p.Hb * R; x += nthreads) p.dbias[(x / R) * p.bias_sh + x % R] = 0.f;
  if (!p.dfreqs) return;
  const int64_t n = (int64_t)p.Bt * p.Ht * p.Nk * R;
  // dense (bt, ht, n, d) layout (the usual one): one flat range
  const bool dense = p.df_s[2] == R && (p.Ht == 1 || p.df_s[1] == (int64_t)p.Nk * R) &&
                     (p.Bt == 1 || p.df_s[0] == (int64_t)p.Ht * p.Nk * R);
  for (int64_t x = gid; x < n; x += nthreads) {
    if (dense) {
      p.dfreqs[x] = 0.f;
    } else {
      const int d = (int)(x % R);
      int64_t rest = x / R;
      const int row = (int)(rest % p.Nk);
      rest /= p.Nk;
      const int ht = (int)(rest % p.Ht), bt = (int)(rest / p.Ht);
      p.dfreqs[(int64_t)bt * p.df_s[0] + (int64_t)ht * p.df_s[1] + (int64_t)row * p.df_s[2] + d] = 0.f;
    }
  }
}

}  // namespace pope
