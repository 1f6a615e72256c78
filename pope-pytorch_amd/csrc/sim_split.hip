// Fused PoPE similarity on bf16 MFMA with split operands (gfx950).
//
// The fp32 products of the similarity (triton_pope.py:28-256; sim.hip for the fp32 MFMA path)
// run here as three bf16 products: every fp32 operand x is split into hi = bf16(x) and
// lo = bf16(x - hi), and a . b = hi_a hi_b + hi_a lo_b + lo_a hi_b (+ lo_a lo_b, dropped, below
// 2^-16 of |a||b|), accumulated in fp32 by v_mfma_f32_32x32x16_bf16.  Operands carry 16
// significant bits: more than the TF32 (10 bits) the reference multiplies in by default
// (allow_tf32=True, triton_pope.py:63,145,224), less than fp32 (24 bits), which the fp32 MFMA
// path keeps for allow_tf32=False.  Per product MAC the bf16 MFMA does 16x the fp32 MFMA rate,
// so the three products take about a fifth of the fp32 time.
//
// Kernels
//   sim_split_prep : the expanded rows Q_hat / K_hat (columns [a cos | a sin | rest], the
//                    reference's rounding of the key phase fl(F_j + bias), pope.py:56) split
//                    into hi / lo bf16 planes, row-major (forward) or transposed (backward);
//   sim_split_fwd  : S = Q_hat K_hat^T, two or four neighbouring 128 x 128 tiles per workgroup;
//   sim_split_uw   : U = G K_hat (u_job: G = dS rows read from HBM and split on the fly) and
//                    W = G^T Q_hat (w_job: G tiles split once per workgroup into LDS, transposed),
//                    in one launch whose job order puts the two reads of each block of G close
//                    together in time.
// The chain rule of the polar transform then runs in sim.hip's finalize kernel on U and W.
#include <type_traits>

#include "pope_common.hpp"
#include "pope_kernels.hpp"
#include "sim_phase.hpp"

namespace pope {

namespace {

constexpr int kThreads = 256;
constexpr int64_t kSimMinJobs = 512;
constexpr int kPrepItems = 2;          // plane preparation items per thread   // U / W workgroups below which each job's reduction is split

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Splits 8 fp32 values into bf16 hi / lo planes (round to nearest even both times).
__device__ __forceinline__ void split8(const float* v, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t h = BF16::pack2(v[2 * s], v[2 * s + 1]);
    hi[s] = h;
    lo[s] = BF16::pack2(v[2 * s] - __uint_as_float(h << 16), v[2 * s + 1] - __uint_as_float(h & 0xffff0000u));
  }
}

__device__ __forceinline__ f32x16 mfma3(u32x4 ah, u32x4 al, u32x4 bh, u32x4 bl, f32x16 c) {
  typedef BF16::vec8 v8;
  c = BF16::mfma32(as_vec8<v8>(al), as_vec8<v8>(bh), c);
  c = BF16::mfma32(as_vec8<v8>(ah), as_vec8<v8>(bl), c);
  return BF16::mfma32(as_vec8<v8>(ah), as_vec8<v8>(bh), c);
}

// Work items per row of the split planes: R / 8 rotated dim groups (each a cos and a sin chunk of
// 8 columns, one phase evaluation for both), then one item per other 8-column chunk (pass-through
// dims, zero padding up to EP).
__host__ __device__ __forceinline__ int prep_items(int EP, int R) { return EP / 8 - R / 8; }

// The split kernels never get phase tables (those are built for the fp32 kernels only): the
// phases are computed in place, theta = F[b, h, n, d] for queries (n = Nk - Nq + i, no bias) and
// fl(F[b, hk, n, d] + bias[hk, d]) for keys (pope.py:56, triton_pope.py:76: the sum rounded to
// fp32 first), then sincos_rev.  Items: (row, 8-column chunk), the query rows of every (b, h)
// first (side 0), then the key rows of every (b, hk) (side 1).  Each thread takes items i, i + T, i + 2T, ... (T threads in
// the grid) with the next item's loads issued before the current item is expanded and stored,
// so the loads, the arithmetic and the stores of the grid overlap instead of running as three
// chip-wide phases.
// transposed = 0: planes (heads, NP, EP); 1: planes (heads, EP, NP), rows fastest over threads so
// that each 2-byte store of a wave covers 64 consecutive rows.
struct PrepItem {
  int side, bh, n, ch;
};
struct PrepIn {
  float4 x0, x1;   // the row's input values at dims [8 ch, 8 ch + 8) (clamped)
  float f[8];      // F at the phase row, rotated dims [8 ch, 8 ch + 8) (clamped)
  float bb[8];     // the key side's bias at those dims
};

__global__ __launch_bounds__(kThreads) void sim_split_prep_kernel(SimParams p, SimSplit sp, int transposed) {
  const int R = p.R, D = p.D, nch = prep_items(p.EP, R);
  const int64_t total0 = (int64_t)p.B * p.Hq * sp.NqP * nch;
  const int64_t total = total0 + (int64_t)p.B * p.Hk * sp.NkP * nch;
  const int64_t T = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (p.zero_grads) sim_clear_grads(p, i, T);   // the backward's first launch
  if (i >= total) return;
  const int q_off = p.Nk - p.Nq;

  auto item = [&](int64_t g) {
    PrepItem it;
    it.side = g < total0 ? 0 : 1;
    const int64_t x = it.side == 0 ? g : g - total0;
    const int NP = it.side == 0 ? sp.NqP : sp.NkP;
    if (total < INT32_MAX) {   // the usual case: 32-bit index decomposition
      const int xi = (int)x;
      if (transposed) {
        it.n = xi % NP;
        const int r = xi / NP;
        it.ch = r % nch;
        it.bh = r / nch;
      } else {
        it.ch = xi % nch;
        const int r = xi / nch;
        it.n = r % NP;
        it.bh = r / NP;
      }
    } else if (transposed) {
      it.n = (int)(x % NP);
      const int64_t r = x / NP;
      it.ch = (int)(r % nch);
      it.bh = (int)(r / nch);
    } else {
      it.ch = (int)(x % nch);
      const int64_t r = x / nch;
      it.n = (int)(r % NP);
      it.bh = (int)(r / NP);
    }
    return it;
  };
  // Branch-free loads at clamped rows and dims: an item past the rows or past D stores zeros.
  auto load = [&](const PrepItem& it) {
    PrepIn in;
    const int heads_h = it.side == 0 ? p.Hq : p.Hk;
    const int N = it.side == 0 ? p.Nq : p.Nk;
    const int hh = it.bh % heads_h, b = it.bh / heads_h;
    const int nn = min(it.n, N - 1);
    const float* x = it.side == 0 ? p.q + (int64_t)b * p.q_s[0] + (int64_t)hh * p.q_s[1] + (int64_t)nn * p.q_s[2]
                                  : p.k + (int64_t)b * p.k_s[0] + (int64_t)hh * p.k_s[1] + (int64_t)nn * p.k_s[2];
    const int dx = min(8 * it.ch, D - 8);
    in.x0 = *reinterpret_cast<const float4*>(x + dx);
    in.x1 = *reinterpret_cast<const float4*>(x + dx + 4);
    if (R > 0) {
      const int d0 = min(8 * it.ch, R - 8);
      const int prow = it.side == 0 ? q_off + nn : nn;
      const float* f = p.freqs + (int64_t)b * p.f_s[0] + (int64_t)hh * p.f_s[1] + (int64_t)prow * p.f_s[2] + d0;
      // the query side reads bias row 0 (always present) and never uses it
      const float* bp = p.bias + (int64_t)(it.side == 1 ? hh : 0) * p.bias_sh + d0;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        in.f[s] = f[s];
        in.bb[s] = bp[s];
      }
    }
    return in;
  };
  auto emit = [&](const PrepItem& it, const PrepIn& in) {
    const int NP = it.side == 0 ? sp.NqP : sp.NkP;
    const int N = it.side == 0 ? p.Nq : p.Nk;
    uint16_t* ph = it.side == 0 ? sp.qh : sp.kh;
    uint16_t* pl = it.side == 0 ? sp.ql : sp.kl;
    auto store = [&](int e0, const float* v) {   // split 8 columns [e0, e0 + 8) of the row
      u32x4 hi, lo;
      split8(v, hi, lo);
      if (!transposed) {
        const int64_t o = ((int64_t)it.bh * NP + it.n) * p.EP + e0;
        *reinterpret_cast<u32x4*>(ph + o) = hi;
        *reinterpret_cast<u32x4*>(pl + o) = lo;
      } else {
        const int64_t o = ((int64_t)it.bh * p.EP + e0) * NP + it.n;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          ph[o + (int64_t)s * NP] = (uint16_t)((s & 1) ? hi[s >> 1] >> 16 : hi[s >> 1] & 0xffffu);
          pl[o + (int64_t)s * NP] = (uint16_t)((s & 1) ? lo[s >> 1] >> 16 : lo[s >> 1] & 0xffffu);
        }
      }
    };
    const bool live = it.n < N;
    const float xv[8] = {in.x0.x, in.x0.y, in.x0.z, in.x0.w, in.x1.x, in.x1.y, in.x1.z, in.x1.w};
    if (8 * it.ch < R) {   // rotated dims d0 .. d0 + 7: cos chunk at column d0, sin chunk at R + d0
      float vc[8], vs[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float th = it.side == 1 ? in.f[s] + in.bb[s] : in.f[s];
        float sn, cs;
        sincos_rev(th, &sn, &cs);
        const float a = live ? softplus_f(xv[s]) : 0.f;
        vc[s] = a * cs;
        vs[s] = a * sn;
      }
      store(8 * it.ch, vc);
      store(R + 8 * it.ch, vs);
    } else {               // pass-through dims (columns < E) or zero padding
      const bool on = live && 8 * it.ch < D;
      float v[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) v[s] = on ? xv[s] : 0.f;
      store(8 * it.ch + R, v);
    }
  };

  PrepItem cur = item(i);
  PrepIn in = load(cur);
  for (;;) {
    const int64_t nx = i + T;
    const PrepItem nxt = item(min(nx, total - 1));
    const PrepIn nin = load(nxt);   // issued before this item's arithmetic and stores
    emit(cur, in);
    if (nx >= total) break;
    i = nx;
    cur = nxt;
    in = nin;
  }
}

// Operand tiles in LDS: [hi, lo plane][128 rows][32 k values + 8 pad] bf16.  The 80-byte row
// stride keeps the 16-byte reads of 16 consecutive rows on distinct banks.  A tile is loaded
// once per workgroup (thread t: chunks t + 256 m, m < 4, of 16 bytes) and read by every wave.
constexpr int kLd = 40;
constexpr int kTile = 2 * 128 * kLd;   // bf16 per tile (both planes)

// Loads rows [0, 128) x k values [k0, k0 + 32) of two planes (row stride rs elements); rows at
// or past nrows (nrows >= 1) repeat the last row.  Such rows only reach output columns that the
// callers never store (expanded columns past EP), and loads without a select on their values
// leave each wait to the instruction that first uses them.
__device__ __forceinline__ void tile_load(const uint16_t* ph, const uint16_t* pl, int64_t rs, int k0, int nrows,
                                          u32x4* v, int tid) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = tid + kThreads * m, plane = c >> 9, row = (c >> 2) & 127, kc = c & 3;
    const uint16_t* base = plane ? pl : ph;
    v[m] = ld16(base + min(row, nrows - 1) * rs + k0 + 8 * kc);
  }
}
__device__ __forceinline__ void tile_store(uint16_t* t, const u32x4* v, int tid) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = tid + kThreads * m, plane = c >> 9, row = (c >> 2) & 127, kc = c & 3;
    *reinterpret_cast<u32x4*>(t + plane * 128 * kLd + row * kLd + 8 * kc) = v[m];
  }
}
// MFMA operand of rows r .. r + 31 (lane = row r + lane % 32), 16-wide k step u: the hi and lo
// planes' 8 values at k = 16 u + 8 (lane / 32).
__device__ __forceinline__ void tile_frag(const uint16_t* t, int r, int u, int lr, int hf, u32x4& hi, u32x4& lo) {
  const int o = (r + lr) * kLd + 16 * u + 8 * hf;
  hi = *reinterpret_cast<const u32x4*>(t + o);
  lo = *reinterpret_cast<const u32x4*>(t + 128 * kLd + o);
}

// Forward: one workgroup = tpw neighbouring 128 x 128 tiles of S (key blocks tpw jp ..
// tpw jp + tpw - 1), computed one after the other; 4 waves of 64 x 64 per tile (2 x 2 blocks of 32 x 32).  Per 32
// expanded columns the Q_hat and K_hat tiles go through LDS.  The steps of all tiles form one
// stream with two steps in flight (LDS buffer (s & 1) holds step s, register set (s + 1) & 1 step
// s + 1, the other set receives step s + 2, clamped to the last step), so a tile's first loads
// overlap the previous tile's products and its S stores.
template <int tpw>
__global__ __launch_bounds__(kThreads, 2) void sim_split_fwd_kernel(SimParams p, SimSplit sp, int nib, int njb) {
  __shared__ __attribute__((aligned(16))) uint16_t ts[2][2][kTile];   // [buffer][Q_hat, K_hat]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int njp = (njb + tpw - 1) / tpw;
  const int jp = id % njp, ib = (id / njp) % nib, bh = id / (njp * nib);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int EP = p.EP;
  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  const int64_t qo = ((int64_t)bh * sp.NqP + ib * 128) * EP;
  const int64_t ko = ((int64_t)(b * p.Hk + hk) * sp.NkP + jp * tpw * 128) * EP;
  const int nst = EP / 32, ntile = min(tpw, njb - tpw * jp), S = ntile * nst;
  // S is written with non-temporal stores: its 4 bytes per (i, j) are not read again by this
  // path, and kept out of the caches they leave the operand planes and dS of the neighbouring
  // launches cached (C2: the step's other kernels ran 10-15 us faster)
  float* sbase = p.sim + (int64_t)b * p.sim_s[0] + (int64_t)h * p.sim_s[1];

  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[x][y][r] = 0.f;

  u32x4 va[2][4], vb[2][4];
  auto fetch = [&](int st, int k) {
    const int sc = min(st, S - 1), t = sc / nst, kk = sc - t * nst;
    tile_load(sp.qh + qo, sp.ql + qo, EP, 32 * kk, 128, va[k], tid);
    const int64_t kt = ko + (int64_t)t * 128 * EP;
    tile_load(sp.kh + kt, sp.kl + kt, EP, 32 * kk, 128, vb[k], tid);
  };
  auto step = [&](int st, auto kc) {
    constexpr int K = decltype(kc)::value;
    fetch(st + 2, K);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      u32x4 ah[2], al[2], bh16[2], bl16[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        tile_frag(ts[K][0], wr + 32 * x, u, lr, hf, ah[x], al[x]);
        tile_frag(ts[K][1], wc + 32 * x, u, lr, hf, bh16[x], bl16[x]);
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) acc[x][y] = mfma3(ah[x], al[x], bh16[y], bl16[y], acc[x][y]);
    }
    tile_store(ts[K ^ 1][0], va[K ^ 1], tid);   // the last step's copy is never read
    tile_store(ts[K ^ 1][1], vb[K ^ 1], tid);
    if ((st + 1) % nst == 0) {   // the tile's last step: write it, start the next from zero
      const int i0 = ib * 128 + wr, j0 = (tpw * jp + st / nst) * 128 + wc;
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) {
          const int j = j0 + 32 * y + lr;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int i = i0 + 32 * x + 8 * (r >> 2) + 4 * hf + (r & 3);
            if (i < p.Nq && j < p.Nk) __builtin_nontemporal_store(acc[x][y][r], sbase + (int64_t)i * p.sim_s[2] + j);
            acc[x][y][r] = 0.f;
          }
        }
    }
    __syncthreads();
  };
  fetch(0, 0);
  fetch(1, 1);
  tile_store(ts[0][0], va[0], tid);
  tile_store(ts[0][1], vb[0], tid);
  __syncthreads();
  int st = 0;
  for (; st + 1 < S; st += 2) {
    step(st, std::integral_constant<int, 0>{});
    step(st + 1, std::integral_constant<int, 1>{});
  }
  if (st < S) step(st, std::integral_constant<int, 0>{});
}

// U[b,h,i,e] = sum_j G[b,h,i,j] K_hat[b,hk,j,e] over all keys, or with nsplit = 2 over half of
// them (the second half into sp.U2: twice the workgroups of one full pass; the finalize adds them).  One workgroup = 128
// query rows x 128 expanded columns; wave w owns rows 32 w .. 32 w + 31 and all four column
// blocks.  Per step of 32 keys the 128 x 32 G tile is loaded coalesced (thread: one 4-key quad of
// four rows), split once into bf16 hi / lo and stored row-major in LDS, where the A operand (lane =
// row, 8 consecutive keys) is one 16-byte read per plane; the B operand comes from the transposed
// K_hat planes (128 columns e x 32 keys), also through LDS.  Two steps of both are in flight: at
// step st the LDS buffers (st - s0) & 1 hold step st, register set (st - s0 + 1) & 1 holds step
// st + 1 (stored to the other buffers at the end of the step) and the other set receives step
// st + 2 (clamped to the last step: the same loads every step, so each wait covers only the
// loads a store needs).
// One job: (part `half` of nsplit, column block ec, query block ib, batch * head bh); gs: two G tiles, ts: two
// K_hat^T tiles.
template <bool VEC>
__device__ __forceinline__ void u_job(const SimParams& p, const SimSplit& sp, float* U, int nsplit, int half, int ec,
                                      int ib, int bh, uint16_t (*gs)[kTile], uint16_t (*ts)[kTile]) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int Nq = p.Nq, Nk = p.Nk, EP = p.EP;
  const float* gb = p.dsim + (int64_t)b * p.sim_s[0] + (int64_t)h * p.sim_s[1];
  const int nst = (Nk + 31) / 32, hst = (nst + nsplit - 1) / nsplit;
  const int s0 = half * hst, s1 = min(nst, s0 + hst);
  const int64_t bo = ((int64_t)(b * p.Hk + hk) * EP + ec * 128) * sp.NkP;
  const int erows = min(128, EP - ec * 128);
  // G loader: thread -> key quad kq (keys 4 kq .. 4 kq + 3 of the step) of rows rr + 32 m, m < 4:
  // a wave's load reads eight 128-byte row pieces
  const int kq = tid & 7, rr = tid >> 3;

  f32x16 acc[4];
#pragma unroll
  for (int y = 0; y < 4; ++y)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[y][r] = 0.f;

  auto load_g = [&](int st, float4* g) {
    const int j = 32 * st + 4 * kq;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int ii = ib * 128 + rr + 32 * m;
      const float* row = gb + (int64_t)min(ii, Nq - 1) * p.sim_s[2];
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (VEC) {
        // 16-byte aligned rows, Nk a multiple of 8: a quad lies wholly inside or wholly past the
        // row (one past it reads the last quad and is zeroed)
        v = *reinterpret_cast<const float4*>(row + min(j, Nk - 4));
        if (ii >= Nq || j >= Nk) v = make_float4(0.f, 0.f, 0.f, 0.f);
      } else if (ii < Nq) {
        v.x = j < Nk ? row[j] : 0.f;
        v.y = j + 1 < Nk ? row[j + 1] : 0.f;
        v.z = j + 2 < Nk ? row[j + 2] : 0.f;
        v.w = j + 3 < Nk ? row[j + 3] : 0.f;
      }
      g[m] = v;
    }
  };
  // split the thread's four quads; one 8-byte store per plane and row
  auto store_g = [&](uint16_t* t, const float4* g) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t h0 = BF16::pack2(g[m].x, g[m].y), h1 = BF16::pack2(g[m].z, g[m].w);
      const uint32_t l0 = BF16::pack2(g[m].x - __uint_as_float(h0 << 16), g[m].y - __uint_as_float(h0 & 0xffff0000u));
      const uint32_t l1 = BF16::pack2(g[m].z - __uint_as_float(h1 << 16), g[m].w - __uint_as_float(h1 & 0xffff0000u));
      const int o = (rr + 32 * m) * kLd + 4 * kq;
      *reinterpret_cast<u32x2*>(t + o) = u32x2{h0, h1};
      *reinterpret_cast<u32x2*>(t + 128 * kLd + o) = u32x2{l0, l1};
    }
  };
  float4 gr[2][4];
  u32x4 vb[2][4];
  auto fetch = [&](int st, int k) {
    const int sc = min(st, s1 - 1);
    load_g(sc, gr[k]);
    tile_load(sp.kh + bo, sp.kl + bo, sp.NkP, 32 * sc, erows, vb[k], tid);
  };
  auto step = [&](int st, auto kc) {
    constexpr int K = decltype(kc)::value;
    fetch(st + 2, K);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      u32x4 ah, al;
      tile_frag(gs[K], 32 * wave, u, lr, hf, ah, al);
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        u32x4 bh16, bl16;
        tile_frag(ts[K], 32 * y, u, lr, hf, bh16, bl16);
        acc[y] = mfma3(ah, al, bh16, bl16, acc[y]);
      }
    }
    store_g(gs[K ^ 1], gr[K ^ 1]);   // the last step's copy is never read
    tile_store(ts[K ^ 1], vb[K ^ 1], tid);
    __syncthreads();
  };
  if (s0 < s1) {
    fetch(s0, 0);
    fetch(s0 + 1, 1);
    store_g(gs[0], gr[0]);
    tile_store(ts[0], vb[0], tid);
    __syncthreads();
    int st = s0;
    for (; st + 1 < s1; st += 2) {
      step(st, std::integral_constant<int, 0>{});
      step(st + 1, std::integral_constant<int, 1>{});
    }
    if (st < s1) step(st, std::integral_constant<int, 0>{});
  }

  float* ub = (half ? sp.U2 : U) + (int64_t)bh * Nq * EP;
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    const int e = ec * 128 + 32 * y + lr;
    if (e >= EP) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ii = ib * 128 + 32 * wave + 8 * (r >> 2) + 4 * hf + (r & 3);
      if (ii < Nq) ub[(int64_t)ii * EP + e] = acc[y][r];
    }
  }
}

// W[b,hk,j,e] = sum_{h in group(hk)} sum_i G[b,h,i,j] Q_hat[b,h,i,e] over the (query head,
// 32-query step) sequence, or with nsplit = 2 over half of it (the second half into sp.W2).  One workgroup = 128 keys x 128
// expanded columns.  Per step the 32 x 128 G tile is loaded coalesced (thread: 4 rows x 4 keys),
// split once and stored key-major in LDS, so the A operand (lane = key, 8 consecutive queries)
// is one 16-byte LDS read per plane; the transposed Q_hat planes (128 columns e x 32 queries)
// go through LDS the same way.  Both double-buffered.  Wave w owns keys 32 w .. 32 w + 31 and
// all four column blocks.
// One job: (part `half` of nsplit, column block ec, key block jb, batch * kv head bhk); gs: two G^T tiles
// (key-major), qs: two Q_hat^T tiles (column-major).
template <bool VEC>
__device__ __forceinline__ void w_job(const SimParams& p, const SimSplit& sp, float* W, int nsplit, int half, int ec,
                                      int jb, int bhk, uint16_t (*gs)[kTile], uint16_t (*qs)[kTile]) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int b = bhk / p.Hk, hk = bhk % p.Hk;
  const int Nq = p.Nq, Nk = p.Nk, EP = p.EP;
  const int groups = p.Hq / p.Hk;
  const int nis = (Nq + 31) / 32;              // 32-query steps per head
  const int nst = groups * nis, hst = (nst + nsplit - 1) / nsplit;
  const int s0 = half * hst, s1 = min(nst, s0 + hst);
  const int erows = min(128, EP - ec * 128);
  // G tile loader: thread -> key quad c (keys 4 c .. 4 c + 3), rows 4 rg .. 4 rg + 3 of the step.
  // rg runs fastest so that the eight lanes of one key quad write one 64-byte LDS row segment:
  // a 16-lane group of 8-byte stores then covers every bank once (80-dword row stride); a wave's
  // global load reads eight 128-byte row segments.
  const int c = tid >> 3, rg = tid & 7;
  const int jq = jb * 128 + 4 * c;

  f32x16 acc[4];
#pragma unroll
  for (int y = 0; y < 4; ++y)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[y][r] = 0.f;

  auto load_g = [&](int st, float4* g) {
    const int h = hk + (st / nis) * p.Hk, i0 = (st % nis) * 32;
    const float* gb = p.dsim + (int64_t)b * p.sim_s[0] + (int64_t)h * p.sim_s[1];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int ii = i0 + 4 * rg + t;
      const float* row = gb + (int64_t)min(ii, Nq - 1) * p.sim_s[2];
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (VEC) {
        // 4-wide and branch-free (16-byte aligned rows, Nk a multiple of 8: a key quad lies wholly
        // inside or wholly past the row; one past it reads the last quad and is zeroed), so the wait
        // before a step's stores covers only that step's loads.  Non-temporal (at C2 the U / W launch
        // and the finalize after it each ran about 1.5 us faster than with these loads cached; the
        // U jobs' loads of G stay cached, which was slower non-temporal)
        v = __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row + min(jq, Nk - 4))));
        if (ii >= Nq || jq >= Nk) v = make_float4(0.f, 0.f, 0.f, 0.f);
      } else if (ii < Nq) {
        v.x = jq < Nk ? row[jq] : 0.f;
        v.y = jq + 1 < Nk ? row[jq + 1] : 0.f;
        v.z = jq + 2 < Nk ? row[jq + 2] : 0.f;
        v.w = jq + 3 < Nk ? row[jq + 3] : 0.f;
      }
      g[t] = v;
    }
  };
  // split the thread's 4 x 4 patch; key s gets 4 consecutive queries: one 8-byte store per plane
  auto store_g = [&](uint16_t* t, const float4* g) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = s == 0 ? g[q].x : s == 1 ? g[q].y : s == 2 ? g[q].z : g[q].w;
      const uint32_t h0 = BF16::pack2(v[0], v[1]), h1 = BF16::pack2(v[2], v[3]);
      const uint32_t l0 = BF16::pack2(v[0] - __uint_as_float(h0 << 16), v[1] - __uint_as_float(h0 & 0xffff0000u));
      const uint32_t l1 = BF16::pack2(v[2] - __uint_as_float(h1 << 16), v[3] - __uint_as_float(h1 & 0xffff0000u));
      const int o = (4 * c + s) * kLd + 4 * rg;
      *reinterpret_cast<u32x2*>(t + o) = u32x2{h0, h1};
      *reinterpret_cast<u32x2*>(t + 128 * kLd + o) = u32x2{l0, l1};
    }
  };
  auto load_q = [&](int st, u32x4* v) {
    const int h = hk + (st / nis) * p.Hk, i0 = (st % nis) * 32;
    const int64_t qo = ((int64_t)(b * p.Hq + h) * EP + ec * 128) * sp.NqP;
    tile_load(sp.qh + qo, sp.ql + qo, sp.NqP, i0, erows, v, tid);
  };
  // Two steps in flight: at step st the LDS buffer (st - s0) & 1 holds step st, register set
  // (st - s0 + 1) & 1 step st + 1 (stored to the other buffer at the end of the step) and the other
  // set receives step st + 2 (clamped to the last step: the same loads every step).
  float4 gr[2][4];
  u32x4 vq[2][4];
  auto fetch = [&](int st, int k) {
    load_g(min(st, s1 - 1), gr[k]);
    load_q(min(st, s1 - 1), vq[k]);
  };
  auto step = [&](int st, auto kc) {
    constexpr int K = decltype(kc)::value;
    fetch(st + 2, K);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      u32x4 ah, al;
      tile_frag(gs[K], 32 * wave, u, lr, hf, ah, al);
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        u32x4 bh16, bl16;
        tile_frag(qs[K], 32 * y, u, lr, hf, bh16, bl16);
        acc[y] = mfma3(ah, al, bh16, bl16, acc[y]);
      }
    }
    store_g(gs[K ^ 1], gr[K ^ 1]);   // the last step's copy is never read
    tile_store(qs[K ^ 1], vq[K ^ 1], tid);
    __syncthreads();
  };
  if (s0 < s1) {
    fetch(s0, 0);
    fetch(s0 + 1, 1);
    store_g(gs[0], gr[0]);
    tile_store(qs[0], vq[0], tid);
    __syncthreads();
    int st = s0;
    for (; st + 1 < s1; st += 2) {
      step(st, std::integral_constant<int, 0>{});
      step(st + 1, std::integral_constant<int, 1>{});
    }
    if (st < s1) step(st, std::integral_constant<int, 0>{});
  }

  float* wb = (half ? sp.W2 : W) + (int64_t)bhk * Nk * EP;
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    const int e = ec * 128 + 32 * y + lr;
    if (e >= EP) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int jj = jb * 128 + 32 * wave + 8 * (r >> 2) + 4 * hf + (r & 3);
      if (jj < Nk) wb[(int64_t)jj * EP + e] = acc[y][r];
    }
  }
}

// Both passes in one launch.  Logical ids run over units of (batch, kv head): a unit holds the U
// jobs of the kv head's query heads and the W jobs of the kv head, interleaved, so the two jobs
// that read a block of G run at about the same time (xcd_remap keeps a unit's jobs on one XCD)
// and the G of the units in flight (16.8 MB per head at 2048 x 2048) fits the 256 MB last-level
// cache between its two reads.  U jobs and W jobs also hide each other's load latency.  The LDS of
// a workgroup is the larger of the two jobs' needs (four tiles, 80 KB; two workgroups per CU).
template <bool VEC>
__global__ __launch_bounds__(kThreads, 2) void sim_split_uw_kernel(SimParams p, SimSplit sp, float* U, float* W,
                                                                   int nib, int njb, int nec, int nsplit) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[4][kTile];
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int groups = p.Hq / p.Hk;
  const int nu = nsplit * nec * nib * groups, nw = nsplit * nec * njb;   // jobs per unit
  const int unit = id / (nu + nw), r = id % (nu + nw);
  const int b = unit / p.Hk, hk = unit % p.Hk;
  const int m = min(nu, nw);
  const bool is_u = r < 2 * m ? !(r & 1) : nu > nw;
  const int k = r < 2 * m ? r >> 1 : r - m;
  const int half = k % nsplit, rest = k / nsplit;
  if (is_u) {
    const int ec = rest % nec, ib = (rest / nec) % nib, g = rest / (nec * nib);
    u_job<VEC>(p, sp, U, nsplit, half, ec, ib, b * p.Hq + g * p.Hk + hk, lds, lds + 2);
  } else {
    w_job<VEC>(p, sp, W, nsplit, half, rest % nec, rest / nec, b * p.Hk + hk, lds, lds + 2);
  }
}

}  // namespace

hipError_t launch_sim_split_prep(const SimParams& p, const SimSplit& sp, int transposed, hipStream_t s) {
  const int64_t total = ((int64_t)p.B * p.Hq * sp.NqP + (int64_t)p.B * p.Hk * sp.NkP) * prep_items(p.EP, p.R);
  // kPrepItems items per thread, so that each thread has a next item's loads in flight
  const int64_t blocks = (total + kThreads * kPrepItems - 1) / (kThreads * kPrepItems);
  return launch_named("sim_split_prep", sim_split_prep_kernel, dim3((unsigned)blocks), dim3(kThreads), s, p, sp,
                      transposed);
}

hipError_t launch_sim_split_fwd(const SimParams& p, const SimSplit& sp, hipStream_t s) {
  hipError_t e = launch_sim_split_prep(p, sp, 0, s);
  if (e != hipSuccess) return e;
  const int nib = (p.Nq + 127) / 128, njb = (p.Nk + 127) / 128;
  // tiles per workgroup: 4 while that still leaves 1,024 workgroups (two rounds at two per CU), else 2
  const int64_t rows = (int64_t)nib * p.B * p.Hq;
  if (rows * ((njb + 3) / 4) >= 1024)
    return launch_named("sim_split_fwd", sim_split_fwd_kernel<4>, dim3((unsigned)(rows * ((njb + 3) / 4))),
                        dim3(kThreads), s, p, sp, nib, njb);
  return launch_named("sim_split_fwd", sim_split_fwd_kernel<2>, dim3((unsigned)(rows * ((njb + 1) / 2))),
                      dim3(kThreads), s, p, sp, nib, njb);
}

hipError_t launch_sim_split_bwd(const SimParams& p, const SimSplit& sp, float* U, float* W, hipStream_t s) {
  hipError_t e = launch_sim_split_prep(p, sp, 1, s);
  if (e != hipSuccess) return e;
  const int nec = (p.EP + 127) / 128;
  const int nib = (p.Nq + 127) / 128, njb = (p.Nk + 127) / 128;
  // each job's reduction split in kSimSplits parts (partial sums U, U2 and W, W2 that the
  // finalize adds) when one part per job would leave fewer than kSimMinJobs workgroups
  const int64_t jobs1 = (int64_t)(nec * nib * (p.Hq / p.Hk) + nec * njb) * p.B * p.Hk;
  const int nsplit = jobs1 < kSimMinJobs ? 2 : 1;
  const dim3 grid((unsigned)(nsplit * jobs1));
  // VEC needs Nk % 8 == 0: every 8-key chunk then lies wholly inside or wholly past the row, so a
  // clamped chunk is only ever one whose entries are all zeroed
  e = p.g_vec && p.Nk % 8 == 0
          ? launch_named("sim_split_uw", sim_split_uw_kernel<true>, grid, dim3(kThreads), s, p, sp, U, W, nib, njb, nec,
                         nsplit)
          : launch_named("sim_split_uw", sim_split_uw_kernel<false>, grid, dim3(kThreads), s, p, sp, U, W, nib, njb, nec,
                         nsplit);
  if (e != hipSuccess) return e;
  return launch_sim_finalize(p, U, nsplit == 2 ? sp.U2 : nullptr, W, nsplit == 2 ? sp.W2 : nullptr, s);
}

}  // namespace pope
