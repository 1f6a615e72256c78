// Shared preparation of the PoPE flash forward and backward (gfx950).
//
// The polar transform of the reference (pope.py:30-86, triton_pope_flash_attn.py:52-57,73-79)
// is applied once per call and the expanded rows are kept in the caller's workspace.  One
// launch, four kinds of blocks:
//   K_hat items   8 dims of one key row: cos/sin(F[n, d]) (FMA-split reduction to revolutions and
//                 the hardware sine / cosine, sincos_rev), the row's cos and sin chunks of K_hat
//                 and, from the items of the first batch / head that own a table row, the
//                 cos/sin table (fp32 pairs, n < Nk) that the backward's chain rule reads;
//   Q_hat items   the same for a query row at phase F[Nk - Nq + i] - bias, pre-scaled by
//                 softmax_scale * log2 e;
//   mask words    bit j of word w: key 64 w + j < Nk and mask[b, key] != 0 (the reference's keep
//                 convention, attention.py:129-131), one wave per word;
//   batch blocks  one past the last visible key of each batch, from the mask bytes directly;
//                 the first one also writes cos/sin(bias) for the backward.
// No block reads what another writes, so nothing orders them.  The forward reads K_hat / Q_hat
// tiles straight into LDS; the backward reuses them (and the tables) when the forward's
// workspace is handed to it.
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(uint16_t* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Block ranges of flash_prep: [K_hat items | Q_hat items | mask words (4 per block) | batches].
struct PrepGrid {
  int nitem;            // work items per row: R/8 rotated chunks, (D-R)/8 pass-through, (EP-E)/8 zero
  int64_t n_k, n_q;     // items of the K_hat and Q_hat parts
  int b_k, b_q, b_mask;
};
PrepGrid prep_grid(const FlashPrep& p) {
  PrepGrid g;
  g.nitem = p.D / 8 + (p.EP - p.D - p.R) / 8;
  g.n_k = (int64_t)p.B * p.Hk * p.NkP * g.nitem;
  g.n_q = (int64_t)p.B * p.Hq * p.NqP * g.nitem;
  g.b_k = (int)((g.n_k + 255) / 256);
  g.b_q = (int)((g.n_q + 255) / 256);
  g.b_mask = (p.B * p.NW + 3) / 4;
  return g;
}

// One work item of an expanded row: x = the 8 raw elements at dim d0 (rotated when d0 < R),
// (cs, sn) their phase cos/sin; writes the cos chunk at column d0 and the sin chunk at R + d0,
// or the raw chunk at R + d0 for a pass-through dim.  `mul` scales every column.
template <typename T>
__device__ __forceinline__ void expand_item(uint16_t* row, int d0, int R, u32x4 raw, const float* cs,
                                           const float* sn, float mul) {
  float x[8];
  unpack8<T>(raw, x);
  if (d0 >= R) {
    u32x4 w;
#pragma unroll
    for (int s = 0; s < 4; ++s) w[s] = T::pack2(x[2 * s] * mul, x[2 * s + 1] * mul);
    st16(row + R + d0, w);
    return;
  }
  u32x4 wc, ws;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float a0 = softplus_f(x[2 * s]) * mul, a1 = softplus_f(x[2 * s + 1]) * mul;
    wc[s] = T::pack2(a0 * cs[2 * s], a1 * cs[2 * s + 1]);
    ws[s] = T::pack2(a0 * sn[2 * s], a1 * sn[2 * s + 1]);
  }
  st16(row + d0, wc);
  st16(row + R + d0, ws);
}

template <typename T>
__global__ __launch_bounds__(256) void flash_prep_kernel(FlashPrep p, PrepGrid g) {
  const int blk = blockIdx.x;
  const int D = p.D, R = p.R, EP = p.EP, E = D + R;
  if (blk >= g.b_k + g.b_q + g.b_mask) {   // batch b: 1 + last visible key; cos/sin(bias)
    const int b = blk - g.b_k - g.b_q - g.b_mask;
    if (b == 0)
      for (int i = threadIdx.x; i < p.Hb * R; i += 256) {
        const int hb = i / R, d = i % R;
        float sn, cs;
        sincos_rev(p.bias[(int64_t)hb * p.bias_sh + d], &sn, &cs);
        p.btab[i] = make_float2(cs, sn);
      }
    int last = 0;
    if (!p.has_mask) {
      last = p.Nk;
    } else {
      const uint8_t* mrow = p.mask + (int64_t)b * p.mask_sb;
      int j = threadIdx.x;   // each thread's keys ascend: its last hit is its maximum
      if ((reinterpret_cast<uintptr_t>(mrow) & 15) == 0) {
        // 16 mask bytes per load; the highest nonzero byte of a word (little-endian) is its last key
        const int n16 = p.Nk / 16;
        for (int c = threadIdx.x; c < n16; c += 256) {
          const u32x4 w = *reinterpret_cast<const u32x4*>(mrow + 16 * c);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (w[t]) last = 16 * c + 4 * t + (31 - (int)__builtin_clz(w[t])) / 8 + 1;
        }
        j = 16 * n16 + threadIdx.x;
      }
      for (; j < p.Nk; j += 256)
        if (mrow[j]) last = j + 1;
    }
    __shared__ int red[256];
    red[threadIdx.x] = last;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
      if ((int)threadIdx.x < st) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + st]);
      __syncthreads();
    }
    if (threadIdx.x == 0) p.kend[b] = red[0];
    return;
  }
  if (blk >= g.b_k + g.b_q) {   // key visibility words: one wave per word, one lane per key
    const int wi = (blk - g.b_k - g.b_q) * 4 + (threadIdx.x >> 6);
    if (wi >= p.B * p.NW) return;
    const int b = wi / p.NW, w = wi % p.NW, lane = threadIdx.x & 63;
    const int key = 64 * w + lane;
    const bool vis = key < p.Nk && (!p.has_mask || p.mask[(int64_t)b * p.mask_sb + key] != 0);
    const uint64_t bits = __ballot(vis);
    if (lane == 0) p.mwords[wi] = bits;
    return;
  }
  const bool is_k = blk < g.b_k;
  const int64_t idx = (int64_t)(is_k ? blk : blk - g.b_k) * 256 + threadIdx.x;
  if (idx >= (is_k ? g.n_k : g.n_q)) return;
  const int NP = is_k ? p.NkP : p.NqP;
  int item, n, bh;
  if (idx < INT32_MAX) {   // the usual case: 32-bit index decomposition
    const int i = (int)idx;
    item = i % g.nitem;
    const int row = i / g.nitem;
    n = row % NP;
    bh = row / NP;
  } else {
    item = (int)(idx % g.nitem);
    const int64_t row = idx / g.nitem;
    n = (int)(row % NP);
    bh = (int)(row / NP);
  }
  const int H = is_k ? p.Hk : p.Hq;
  const int b = bh / H, h = bh % H;
  uint16_t* out = (is_k ? p.kh : p.qh) + ((int64_t)bh * NP + n) * EP;
  const int nvalid = is_k ? p.Nk : p.Nq;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  if (item >= D / 8) {   // zero padding columns [E, EP)
    st16(out + E + 8 * (item - D / 8), zero);
    return;
  }
  const int d0 = 8 * item;
  if (n >= nvalid) {   // padding rows
    if (d0 < R) st16(out + d0, zero);
    st16(out + R + d0, zero);
    return;
  }
  const uint16_t* src = is_k ? p.k + (int64_t)b * p.k_s[0] + (int64_t)h * p.k_s[1] + (int64_t)n * p.k_s[2]
                             : p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1] + (int64_t)n * p.q_s[2];
  const u32x4 raw = ld16(src + d0);
  float cs[8], sn[8];
  if (d0 < R) {
    // phase row: keys use F[j]; queries F[Nk - Nq + i] rotated by -bias of their kv head.  The
    // table and the freqs rows share their (batch, head) selection (Bt, Ht of 1 broadcast).
    const int pos = is_k ? n : p.Nk - p.Nq + n;
    const int bt = p.Bt > 1 ? b : 0, ht = p.Ht > 1 ? h : 0;
    const float* f = p.freqs + (int64_t)bt * p.f_s[0] + (int64_t)ht * p.f_s[1] + (int64_t)pos * p.f_s[2] + d0;
    float x[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) x[t] = f[t];
#pragma unroll
    for (int t = 0; t < 8; ++t) sincos_rev(x[t], &sn[t], &cs[t]);
    if (is_k && (p.Bt > 1 || b == 0) && (p.Ht > 1 || h == 0)) {   // one writer per table row
      float4* tdst = reinterpret_cast<float4*>(p.table + (int64_t)bt * p.t_sb + (int64_t)ht * p.t_sh +
                                               (int64_t)n * R + d0);
#pragma unroll
      for (int t = 0; t < 4; ++t) tdst[t] = make_float4(cs[2 * t], sn[2 * t], cs[2 * t + 1], sn[2 * t + 1]);
    }
    if (!is_k) {
      const int hb = p.Hb > 1 ? h % p.Hk : 0;
      const float* bb = p.bias + (int64_t)hb * p.bias_sh + d0;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        float sb, cb;   // cos(F - b) = cF cb + sF sb,  sin(F - b) = sF cb - cF sb
        sincos_rev(bb[t], &sb, &cb);
        const float c2 = fmaf(cs[t], cb, sn[t] * sb);
        const float s2 = fmaf(sn[t], cb, -cs[t] * sb);
        cs[t] = c2;
        sn[t] = s2;
      }
    }
  }
  expand_item<T>(out, d0, R, raw, cs, sn, is_k ? 1.f : p.qscale);
}

}  // namespace

hipError_t launch_flash_prep(const FlashPrep& p, int dtype, hipStream_t s) {
  const PrepGrid pg = prep_grid(p);
  const dim3 grid(pg.b_k + pg.b_q + pg.b_mask + p.B);
  return dtype == 2 ? launch_named("flash_prep", flash_prep_kernel<BF16>, grid, dim3(256), s, p, pg)
                    : launch_named("flash_prep", flash_prep_kernel<F16>, grid, dim3(256), s, p, pg);
}

}  // namespace pope
