// Shared preparation of the PoPE flash forward and backward (gfx950).
//
// The polar transform of the reference (pope.py:30-86, triton_pope_flash_attn.py:52-57,73-79)
// is applied once per call and the expanded rows are kept in the caller's workspace:
//   flash_setup  cos/sin(F[n, d]) for n < Nk (accurate sincosf, fp32 pairs), cos/sin(bias[hb, d])
//                and the key visibility words (bit j of word w: key 64 w + j < Nk and
//                mask[b, key] != 0, the reference's keep convention, attention.py:129-131);
//   flash_prep   K_hat, Q_hat (pre-scaled by softmax_scale * log2 e) and, per batch, one past
//                the last visible key.
// The forward reads K_hat / Q_hat tiles straight into LDS; the backward reuses them (and the
// cos/sin table for its chain rule) when the forward's workspace is handed to it.
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(uint16_t* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

constexpr int kSetupBlocksMax = 2048;

// Block ranges of flash_setup: [table | bias table | mask words (4 per block, one per wave)].
struct SetupGrid {
  int64_t n_tab;
  int b_tab, b_bias, b_mask;
};
SetupGrid setup_grid(const FlashPrep& p) {
  SetupGrid g;
  g.n_tab = (int64_t)p.Bt * p.Ht * p.Nk * p.R;
  const int64_t bt = (g.n_tab / 4 + 255) / 256;   // four entries per thread
  g.b_tab = (int)(bt > kSetupBlocksMax ? kSetupBlocksMax : bt);
  g.b_bias = p.R > 0 ? (p.Hb * p.R + 255) / 256 : 0;
  g.b_mask = (p.B * p.NW + 3) / 4;
  return g;
}

__global__ __launch_bounds__(256) void flash_setup_kernel(FlashPrep p, SetupGrid g) {
  const int blk = blockIdx.x;
  if (blk < g.b_tab) {
    // cos/sin(F) rows, grid-stride over (bt, ht, n, d): four consecutive entries of one row per
    // thread (R is a multiple of 8), four independent loads, two 16-byte stores; the index is
    // decomposed in 32 bits when the table allows
    for (int64_t i4 = 4 * ((int64_t)blk * 256 + threadIdx.x); i4 < g.n_tab; i4 += 4 * (int64_t)g.b_tab * 256) {
      int d, n, ht, bt;
      if (g.n_tab < INT32_MAX) {
        const int i = (int)i4;
        d = i % p.R;
        int rest = i / p.R;
        n = rest % p.Nk;
        rest /= p.Nk;
        ht = rest % p.Ht;
        bt = rest / p.Ht;
      } else {
        d = (int)(i4 % p.R);
        int64_t rest = i4 / p.R;
        n = (int)(rest % p.Nk);
        rest /= p.Nk;
        ht = (int)(rest % p.Ht);
        bt = (int)(rest / p.Ht);
      }
      const float* f = p.freqs + (int64_t)bt * p.f_s[0] + (int64_t)ht * p.f_s[1] + (int64_t)n * p.f_s[2] + d;
      float x[4], sn[4], cs[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) x[t] = f[t];
#pragma unroll
      for (int t = 0; t < 4; ++t) sincos_acc(x[t], &sn[t], &cs[t]);
      float4* dst = reinterpret_cast<float4*>(p.table + i4);
      dst[0] = make_float4(cs[0], sn[0], cs[1], sn[1]);
      dst[1] = make_float4(cs[2], sn[2], cs[3], sn[3]);
    }
    return;
  }
  if (blk < g.b_tab + g.b_bias) {   // cos/sin(bias)
    const int idx = (blk - g.b_tab) * 256 + threadIdx.x;
    if (idx < p.Hb * p.R) {
      const int hb = idx / p.R, d = idx % p.R;
      float sn, cs;
      sincos_acc(p.bias[(int64_t)hb * p.bias_sh + d], &sn, &cs);
      p.btab[idx] = make_float2(cs, sn);
    }
    return;
  }
  // key visibility words: one wave per word, one lane per key
  const int wi = (blk - g.b_tab - g.b_bias) * 4 + (threadIdx.x >> 6);
  if (wi >= p.B * p.NW) return;
  const int b = wi / p.NW, w = wi % p.NW, lane = threadIdx.x & 63;
  const int key = 64 * w + lane;
  const bool vis = key < p.Nk && (!p.has_mask || p.mask[(int64_t)b * p.mask_sb + key] != 0);
  const uint64_t bits = __ballot(vis);
  if (lane == 0) p.mwords[wi] = bits;
}

// Block ranges of flash_prep: [K_hat items | Q_hat items | kend (one block per batch)].
struct PrepGrid {
  int nitem;            // work items per row: R/8 rotated chunks, (D-R)/8 pass-through, (EP-E)/8 zero
  int64_t n_k, n_q;     // items of the K_hat and Q_hat parts
  int b_k, b_q;
};
PrepGrid prep_grid(const FlashPrep& p) {
  PrepGrid g;
  g.nitem = p.D / 8 + (p.EP - p.D - p.R) / 8;
  g.n_k = (int64_t)p.B * p.Hk * p.NkP * g.nitem;
  g.n_q = (int64_t)p.B * p.Hq * p.NqP * g.nitem;
  g.b_k = (int)((g.n_k + 255) / 256);
  g.b_q = (int)((g.n_q + 255) / 256);
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
  if (blk >= g.b_k + g.b_q) {   // kend: 1 + last visible key of batch b
    const int b = blk - g.b_k - g.b_q;
    int last = 0;
    for (int w = threadIdx.x; w < p.NW; w += 256) {
      const uint64_t bits = p.mwords[(int64_t)b * p.NW + w];
      if (bits) last = max(last, 64 * w + 64 - (int)__builtin_clzll(bits));
    }
    __shared__ int red[256];
    red[threadIdx.x] = last;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
      if ((int)threadIdx.x < s) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + s]);
      __syncthreads();
    }
    if (threadIdx.x == 0) p.kend[b] = red[0];
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
    // phase row: keys use F[j]; queries F[Nk - Nq + i] rotated by -bias of their kv head
    const int pos = is_k ? n : p.Nk - p.Nq + n;
    const float2* t = p.table + (int64_t)b * p.t_sb + (int64_t)h * p.t_sh + (int64_t)pos * R + d0;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float2 f = t[s];
      cs[s] = f.x;
      sn[s] = f.y;
    }
    if (!is_k) {
      const int hb = p.Hb > 1 ? h % p.Hk : 0;
      const float2* bt = p.btab + hb * R + d0;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float2 c = bt[s];   // cos(F - b) = cF cb + sF sb,  sin(F - b) = sF cb - cF sb
        const float c2 = fmaf(cs[s], c.x, sn[s] * c.y);
        const float s2 = fmaf(sn[s], c.x, -cs[s] * c.y);
        cs[s] = c2;
        sn[s] = s2;
      }
    }
  }
  expand_item<T>(out, d0, R, raw, cs, sn, is_k ? 1.f : p.qscale);
}

}  // namespace

hipError_t launch_flash_prep(const FlashPrep& p, int dtype, hipStream_t s) {
  const SetupGrid sg = setup_grid(p);
  const int sblocks = sg.b_tab + sg.b_bias + sg.b_mask;
  hipError_t e = launch_named("flash_setup", flash_setup_kernel, dim3(sblocks), dim3(256), s, p, sg);
  if (e != hipSuccess) return e;
  const PrepGrid pg = prep_grid(p);
  const dim3 grid(pg.b_k + pg.b_q + p.B);
  return dtype == 2 ? launch_named("flash_prep", flash_prep_kernel<BF16>, grid, dim3(256), s, p, pg)
                    : launch_named("flash_prep", flash_prep_kernel<F16>, grid, dim3(256), s, p, pg);
}

}  // namespace pope
