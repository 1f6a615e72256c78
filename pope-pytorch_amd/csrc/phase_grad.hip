// Deterministic phase gradients: fixed-order sums of per-row partial derivatives (gfx950).
//
// The backward kernels of the flash attention, the similarity and the polar transform add the
// phase derivatives into dfreqs / dbias with fp32 atomics by default, so the low bits of those
// sums depend on the order the atomics land in.  In deterministic mode they instead write each
// derivative once, without atomics: the key side's dpsi[b, hk, n, d] (n < Nk) and the query
// side's dphi[b, h, i, d] (i < Nq; its phase row is Nk - Nq + i).  These kernels then sum them in
// a fixed order, so two identical calls give bitwise-equal results:
//   dfreqs[bt, ht, n, d] (+)= sum over b of the batch group of bt of
//                               ( sum over the kv heads of ht of dpsi[b, hk, n, d]
//                               + sum over the query heads of ht of dphi[b, h, n - Nk + Nq, d] )
//   dbias[hb, d] (+)= sum over b, the kv heads of hb and n < Nk of dpsi[b, hk, n, d]
// (a 2-D table's row gathers every batch and head; a per-batch table its batch's heads; a per-head
// table one head).  The bias is a key-side phase offset, so its derivative is the summed key-phase
// derivative (pope.py:56; triton_pope_flash_attn.py:210 adds the same quantity).
// dbias is summed in two passes: kSplits fixed slices of the keys, then the slices in order.
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kSplits = 64;

__global__ __launch_bounds__(256) void dfreqs_reduce_kernel(PhaseGradParams p) {
  const int64_t total = (int64_t)p.Bt * p.Ht * p.Nk * p.R;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int d = (int)(idx % p.R);
  int64_t rest = idx / p.R;
  const int n = (int)(rest % p.Nk);
  rest /= p.Nk;
  const int ht = (int)(rest % p.Ht), bt = (int)(rest / p.Ht);
  const int b0 = p.Bt > 1 ? bt : 0, b1 = p.Bt > 1 ? bt + 1 : p.B;
  const int k0 = p.Ht > 1 ? ht : 0, k1 = p.Ht > 1 ? ht + 1 : p.Hk;
  const int q0 = p.Ht > 1 ? ht : 0, q1 = p.Ht > 1 ? ht + 1 : p.Hq;
  const int i = n - (p.Nk - p.Nq);   // query row whose phase row is n
  float s = 0.f;
  for (int b = b0; b < b1; ++b) {
    if (p.kpart)
      for (int hk = k0; hk < k1; ++hk) s += p.kpart[(((int64_t)b * p.Hk + hk) * p.Nk + n) * p.R + d];
    if (p.qpart && i >= 0)
      for (int h = q0; h < q1; ++h) s += p.qpart[(((int64_t)b * p.Hq + h) * p.Nq + i) * p.R + d];
  }
  float* dst = p.dfreqs + (int64_t)bt * p.df_s[0] + (int64_t)ht * p.df_s[1] + (int64_t)n * p.df_s[2] + d;
  *dst = p.overwrite ? s : *dst + s;
}

// Pass 1: workgroup (bias row hb, 64-dim block, key slice) sums its slice of the keys for every
// (batch, kv head) of hb, lanes over dims, four row phases per workgroup, in a fixed order.
__global__ __launch_bounds__(256) void dbias_slices_kernel(PhaseGradParams p) {
  __shared__ float red[4][64];
  const int dblocks = (p.R + 63) / 64;
  const int slice = blockIdx.x % kSplits;
  const int rest = blockIdx.x / kSplits;
  const int dblk = rest % dblocks, hb = rest / dblocks;
  const int dl = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int d = 64 * dblk + dl;
  const int per = (p.Nk + kSplits - 1) / kSplits;
  const int n0 = slice * per, n1 = min(p.Nk, n0 + per);
  const int k0 = p.Hb > 1 ? hb : 0, k1 = p.Hb > 1 ? hb + 1 : p.Hk;
  float s = 0.f;
  if (d < p.R)
    for (int b = 0; b < p.B; ++b)
      for (int hk = k0; hk < k1; ++hk) {
        const float* kp = p.kpart + ((int64_t)b * p.Hk + hk) * p.Nk * p.R + d;
        for (int n = n0 + ph; n < n1; n += 4) s += kp[(int64_t)n * p.R];
      }
  red[ph][dl] = s;
  __syncthreads();
  if (ph == 0 && d < p.R)
    p.bslices[((int64_t)hb * p.R + d) * kSplits + slice] = ((red[0][dl] + red[1][dl]) + red[2][dl]) + red[3][dl];
}

// Pass 2: one thread per (hb, d) adds the slices in order.
__global__ __launch_bounds__(256) void dbias_finish_kernel(PhaseGradParams p) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= p.Hb * p.R) return;
  const int hb = idx / p.R, d = idx % p.R;
  const float* src = p.bslices + (int64_t)idx * kSplits;
  float s = 0.f;
  for (int k = 0; k < kSplits; ++k) s += src[k];
  float* dst = p.dbias + (int64_t)hb * p.bias_sh + d;
  *dst = p.overwrite ? s : *dst + s;
}

}  // namespace

size_t phase_grad_slices(int Hb, int R) { return (size_t)Hb * R * kSplits; }

hipError_t launch_phase_grad_reduce(const PhaseGradParams& p, hipStream_t s) {
  if (p.R == 0) return hipSuccess;
  if (p.dfreqs) {
    const int64_t total = (int64_t)p.Bt * p.Ht * p.Nk * p.R;
    hipError_t e = launch_named("phase_grad_dfreqs", dfreqs_reduce_kernel, dim3((unsigned)((total + 255) / 256)),
                                dim3(256), s, p);
    if (e != hipSuccess) return e;
  }
  if (p.dbias) {
    const int dblocks = (p.R + 63) / 64;
    hipError_t e = launch_named("phase_grad_dbias", dbias_slices_kernel, dim3(p.Hb * dblocks * kSplits), dim3(256),
                                s, p);
    if (e != hipSuccess) return e;
    return launch_named("phase_grad_dbias_finish", dbias_finish_kernel, dim3((p.Hb * p.R + 255) / 256), dim3(256),
                        s, p);
  }
  return hipSuccess;
}

}  // namespace pope
