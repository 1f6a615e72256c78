// Fused PoPE similarity, fp32 on MFMA (v_mfma_f32_32x32x2f32), gfx950.
//
// Reference: PoPESimilarityFunction (triton_pope.py:258-362) with kernels
// _fwd_kernel :28-83, _bwd_kernel_dqk_df :85-194, _bwd_kernel_dbias_optimized
// :196-256; PyTorch path attention.py:30-47.
//
//   S[b,h,i,j] = sum_e Q_hat[i,e] K_hat[j,e]     (unscaled, fp32)
// with the expanded columns of pope_common.hpp.  The phases come from the
// per-call tables: the key table holds cos/sin(fl(F_j + bias)) exactly as the
// reference rounds it (pope.py:56), the query table cos/sin(F_{q_off+i}).
//
// Backward (G = dS):
//   U = G K_hat (Nq x E),  W = G^T Q_hat (Nk x E)  -- two MFMA passes that read
//   G straight from HBM into registers, writing U and W (fp32) to workspace;
//   a finalize kernel applies the chain rule of the polar transform:
//   dq = sigmoid(q) (cos phi U_c + sin phi U_s), dq_rest = U_rest,
//   dphi = a (cos phi U_s - sin phi U_c)  -> dfreqs rows q_off + i,
//   dk = sigmoid(k) (cos psi W_c + sin psi W_s), dk_rest = W_rest,
//   dpsi = c (cos psi W_s - sin psi W_c)  -> dfreqs rows j and dbias (sum over j).
// dbias = sum_j dpsi replaces the reference's third pass over dS
// (_bwd_kernel_dbias_optimized): both are the derivative of S by the key phase.
#include "pope_common.hpp"
#include "pope_kernels.hpp"
#include "sim_phase.hpp"

namespace pope {

namespace {

constexpr int kThreads = 256;
constexpr int kEC = 32;     // expanded columns per forward chunk
constexpr int kLdsRow = kEC + 4;  // fp32 row stride of the forward chunk buffers

// Transforms 8 consecutive expanded columns [e0, e0+8) of one row into out[8].
// x: the row of q or k (fp32), tab: the row of the phase table (or null when R == 0).
__device__ __forceinline__ void expand8(const float* x, const float2* tab, int e0, int R, int E, bool valid,
                                        float* out) {
  if (!valid || e0 >= E) {
#pragma unroll
    for (int s = 0; s < 8; ++s) out[s] = 0.f;
    return;
  }
  const bool is_cos = e0 < R, is_sin = !is_cos && e0 < 2 * R;
  const int d0 = is_cos ? e0 : e0 - R;
  const float4 x0 = *reinterpret_cast<const float4*>(x + d0);
  const float4 x1 = *reinterpret_cast<const float4*>(x + d0 + 4);
  const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  if (is_cos || is_sin) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float2 cs = tab[d0 + s];
      out[s] = softplus_f(xv[s]) * (is_cos ? cs.x : cs.y);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) out[s] = xv[s];
  }
}

// ---------------------------------------------------------------------------
// Forward: one workgroup = 128 x 128 tile of S; 4 waves of 64 x 64 (2 x 2
// MFMA blocks).  The expanded axis is swept in chunks of 32 columns, each
// chunk transformed into LDS for both operands.
__global__ __launch_bounds__(kThreads, 2) void sim_fwd_kernel(SimParams p, int nib, int njb) {
  __shared__ __attribute__((aligned(16))) float qs[128 * kLdsRow];
  __shared__ __attribute__((aligned(16))) float ks[128 * kLdsRow];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int jb = id % njb, ib = (id / njb) % nib, bh = id / (njb * nib);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int R = p.R, E = p.E, Nq = p.Nq, Nk = p.Nk, q_off = Nk - Nq;
  const int i0 = ib * 128, j0 = jb * 128;
  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;

  // Transform ownership: thread -> (row, 16-column half of the chunk).
  const int trow = tid >> 1, thalf = tid & 1;
  const int qi = i0 + trow, kj = j0 + trow;
  const bool qv = qi < Nq, kv = kj < Nk;
  const float* qrow = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1] + (int64_t)min(qi, Nq - 1) * p.q_s[2];
  const float* krow = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1] + (int64_t)min(kj, Nk - 1) * p.k_s[2];
  const float2* qtab = R ? p.qtab + (int64_t)b * p.qt_sb + (int64_t)h * p.qt_sh + (int64_t)(q_off + min(qi, Nq - 1)) * R
                         : nullptr;
  const float2* ktab = R ? p.ktab + (int64_t)b * p.kt_sb + (int64_t)hk * p.kt_sh + (int64_t)min(kj, Nk - 1) * R
                         : nullptr;

  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[x][y][r] = 0.f;

  for (int c0 = 0; c0 < p.EP; c0 += kEC) {
    __syncthreads();
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int e0 = c0 + 16 * thalf + 8 * g;
      float o[8];
      expand8(qrow, qtab, e0, R, E, qv, o);
      float* dst = &qs[trow * kLdsRow + 16 * thalf + 8 * g];
      *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
      expand8(krow, ktab, e0, R, E, kv, o);
      dst = &ks[trow * kLdsRow + 16 * thalf + 8 * g];
      *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
    }
    __syncthreads();
    // k-slot (t, hf) <-> chunk column 16*hf + t, read 4 at a time.
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) {
      float4 a[2], bb[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        a[x] = *reinterpret_cast<const float4*>(&qs[(wr + 32 * x + lr) * kLdsRow + 16 * hf + 4 * t4]);
        bb[x] = *reinterpret_cast<const float4*>(&ks[(wc + 32 * x + lr) * kLdsRow + 16 * hf + 4 * t4]);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y)
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[x][s], bb[y][s], acc[x][y], 0, 0, 0);
    }
  }
  // S^T layout: acc lane = key column (lr), registers = query rows.
  // Here A = Q (rows i) and B = K (cols j): result lane <-> j, regs <-> i.
  // non-temporal stores: S is not read again by this path and stays out of the caches
  float* sbase = p.sim + (int64_t)b * p.sim_s[0] + (int64_t)h * p.sim_s[1];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int j = j0 + wc + 32 * y + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wr + 32 * x + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (i < Nq && j < Nk) __builtin_nontemporal_store(acc[x][y][r], sbase + (int64_t)i * p.sim_s[2] + j);
      }
    }
}

// ---------------------------------------------------------------------------
// Backward pass A:  U[b,h,i,e] = sum_j G[b,h,i,j] K_hat[b,hk,j,e]
// one workgroup = 128 query rows x 128 expanded columns (chunk ec); 4 waves of
// 32 rows.  G rows go straight from HBM into A-operand registers
// (k-slot (t, hf) <-> key j0 + 32*hf + t).
constexpr int kBJ = 64;
constexpr int kKtRow = 128 + 1;   // fp32 row stride of the K_hat tile (keys x 128 cols)

__global__ __launch_bounds__(kThreads, 2) void sim_bwd_u_kernel(SimParams p, float* U, int nib, int nec) {
  __shared__ float kt[kBJ * kKtRow];
  if (p.zero_grads)   // the backward's first launch
    sim_clear_grads(p, (int64_t)blockIdx.x * kThreads + threadIdx.x, (int64_t)gridDim.x * kThreads);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int ec = id % nec, ib = (id / nec) % nib, bh = id / (nec * nib);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int R = p.R, E = p.E, Nq = p.Nq, Nk = p.Nk;
  const int i = ib * 128 + wave * 32 + lr;
  const int e_base = ec * 128;
  const float* grow = p.dsim + (int64_t)b * p.sim_s[0] + (int64_t)h * p.sim_s[1] + (int64_t)min(i, Nq - 1) * p.sim_s[2];

  f32x16 acc[4];
#pragma unroll
  for (int y = 0; y < 4; ++y)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[y][r] = 0.f;

  // K tile transform ownership: thread -> (key row, 32-column quarter)
  const int trow = tid >> 2, tq = tid & 3;
  const float* kb = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1];
  const float2* tb = R ? p.ktab + (int64_t)b * p.kt_sb + (int64_t)hk * p.kt_sh : nullptr;

  for (int j0 = 0; j0 < Nk; j0 += kBJ) {
    __syncthreads();
    {
      const int kj = j0 + trow;
      const bool kv = kj < Nk;
      const float* krow = kb + (int64_t)min(kj, Nk - 1) * p.k_s[2];
      const float2* ktab = R ? tb + (int64_t)min(kj, Nk - 1) * R : nullptr;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float o[8];
        expand8(krow, ktab, e_base + 32 * tq + 8 * g, R, E, kv, o);
#pragma unroll
        for (int s = 0; s < 8; ++s) kt[trow * kKtRow + 32 * tq + 8 * g + s] = o[s];
      }
    }
    __syncthreads();
    if (p.g_vec && j0 + kBJ <= Nk) {
      // every key of the block in range: the lane's 8 loads issued before the products (rows
      // past Nq read the last row and are never stored)
      float4 gr[8];
#pragma unroll
      for (int t4 = 0; t4 < 8; ++t4) gr[t4] = *reinterpret_cast<const float4*>(grow + j0 + 32 * hf + 4 * t4);
#pragma unroll
      for (int t4 = 0; t4 < 8; ++t4) {
        const float gv[4] = {gr[t4].x, gr[t4].y, gr[t4].z, gr[t4].w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int jr = 32 * hf + 4 * t4 + s;
#pragma unroll
          for (int y = 0; y < 4; ++y)
            acc[y] = __builtin_amdgcn_mfma_f32_32x32x2f32(gv[s], kt[jr * kKtRow + 32 * y + lr], acc[y], 0, 0, 0);
        }
      }
      continue;
    }
#pragma unroll
    for (int t4 = 0; t4 < 8; ++t4) {
      float4 g4 = make_float4(0.f, 0.f, 0.f, 0.f);
      const int jj = j0 + 32 * hf + 4 * t4;
      if (p.g_vec && i < Nq && jj + 3 < Nk) {
        g4 = *reinterpret_cast<const float4*>(grow + jj);
      } else if (i < Nq) {
        float tmp[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) tmp[s] = jj + s < Nk ? grow[jj + s] : 0.f;
        g4 = make_float4(tmp[0], tmp[1], tmp[2], tmp[3]);
      }
      const float gv[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int jr = 32 * hf + 4 * t4 + s;
#pragma unroll
        for (int y = 0; y < 4; ++y)
          acc[y] = __builtin_amdgcn_mfma_f32_32x32x2f32(gv[s], kt[jr * kKtRow + 32 * y + lr], acc[y], 0, 0, 0);
      }
    }
  }
  // result lane <-> column e (B operand lane), regs <-> row i
  float* ub = U + ((int64_t)b * p.Hq + h) * Nq * p.EP;
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    const int e = e_base + 32 * y + lr;
    if (e >= p.EP) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ii = ib * 128 + wave * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
      if (ii < Nq) ub[(int64_t)ii * p.EP + e] = acc[y][r];
    }
  }
}

// Backward pass B:  W[b,hk,j,e] = sum_{h in group(hk)} sum_i G[b,h,i,j] Q_hat[b,h,i,e]
// one workgroup = 128 keys x 128 expanded columns; wave w owns the 32 columns 32 w .. 32 w + 31
// for all 128 keys.  Each lane loads four consecutive keys of a G row at once (16 bytes,
// coalesced over the row): component s of lane l is key 4 l + s, so the four components feed
// four MFMA row blocks whose rows are the keys 4 l + s -- no transposition of G is needed.
// The B operand (Q_hat row i, column e) comes from the transformed tile in LDS.
constexpr int kBI = 64;

__global__ __launch_bounds__(kThreads, 2) void sim_bwd_w_kernel(SimParams p, float* W, int njb, int nec) {
  __shared__ float qt[kBI * kKtRow];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int ec = id % nec, jb = (id / nec) % njb, bhk = id / (nec * njb);
  const int b = bhk / p.Hk, hk = bhk % p.Hk;
  const int R = p.R, E = p.E, Nq = p.Nq, Nk = p.Nk, q_off = Nk - Nq;
  const int j4 = jb * 128 + 4 * lr;   // the lane's four keys
  const bool vec = p.g_vec && j4 + 3 < Nk;
  // every key of the workgroup in range and 16-byte rows: branch-free batched loads
  const bool fast = p.g_vec && jb * 128 + 127 < Nk;
  const int e_base = ec * 128;
  const int groups = p.Hq / p.Hk;

  f32x16 acc[4];
#pragma unroll
  for (int y = 0; y < 4; ++y)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[y][r] = 0.f;

  const int trow = tid >> 2, tq = tid & 3;
  for (int g = 0; g < groups; ++g) {
    const int h = hk + g * p.Hk;
    const float* gb = p.dsim + (int64_t)b * p.sim_s[0] + (int64_t)h * p.sim_s[1];
    const float* qb = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1];
    const float2* tb = R ? p.qtab + (int64_t)b * p.qt_sb + (int64_t)h * p.qt_sh : nullptr;
    for (int i0 = 0; i0 < Nq; i0 += kBI) {
      __syncthreads();
      {
        const int qi = i0 + trow;
        const bool qv = qi < Nq;
        const float* qrow = qb + (int64_t)min(qi, Nq - 1) * p.q_s[2];
        const float2* qtab = R ? tb + (int64_t)(q_off + min(qi, Nq - 1)) * R : nullptr;
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
          float o[8];
          expand8(qrow, qtab, e_base + 32 * tq + 8 * gg, R, E, qv, o);
#pragma unroll
          for (int s = 0; s < 8; ++s) qt[trow * kKtRow + 32 * tq + 8 * gg + s] = o[s];
        }
      }
      __syncthreads();
      if (fast) {
        // 16 rows of G per batch, all loads issued before the products (rows past Nq read the
        // last row; their Q_hat rows are zero).  Row offsets fit 32 bits per (batch, head).
        const float* g0 = gb + j4;
        const int rs = (int)p.sim_s[2];
#pragma unroll
        for (int tc = 0; tc < 32; tc += 16) {
          float4 gr[16];
#pragma unroll
          for (int u = 0; u < 16; ++u)
            gr[u] = *reinterpret_cast<const float4*>(g0 + (uint32_t)(min(i0 + 32 * hf + tc + u, Nq - 1) * rs));
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            const float bq = qt[(32 * hf + tc + u) * kKtRow + 32 * wave + lr];
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(gr[u].x, bq, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(gr[u].y, bq, acc[1], 0, 0, 0);
            acc[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(gr[u].z, bq, acc[2], 0, 0, 0);
            acc[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(gr[u].w, bq, acc[3], 0, 0, 0);
          }
        }
        continue;
      }
#pragma unroll 8
      for (int t = 0; t < 32; ++t) {
        const int ii = i0 + 32 * hf + t;   // k-slot (t, hf)
        float4 g4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ii < Nq) {
          const float* grow = gb + (int64_t)ii * p.sim_s[2];
          if (vec) {
            g4 = *reinterpret_cast<const float4*>(grow + j4);
          } else {
            g4.x = j4 < Nk ? grow[j4] : 0.f;
            g4.y = j4 + 1 < Nk ? grow[j4 + 1] : 0.f;
            g4.z = j4 + 2 < Nk ? grow[j4 + 2] : 0.f;
            g4.w = j4 + 3 < Nk ? grow[j4 + 3] : 0.f;
          }
        }
        const float bq = qt[(32 * hf + t) * kKtRow + 32 * wave + lr];
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(g4.x, bq, acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(g4.y, bq, acc[1], 0, 0, 0);
        acc[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(g4.z, bq, acc[2], 0, 0, 0);
        acc[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(g4.w, bq, acc[3], 0, 0, 0);
      }
    }
  }
  // result lane <-> column e, register r <-> row 8 (r / 4) + 4 hf + r % 4 of block s, i.e. key
  // 4 row + s
  const int e = e_base + 32 * wave + lr;
  if (e < p.EP) {
    float* wb = W + ((int64_t)b * p.Hk + hk) * Nk * p.EP;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int jj = jb * 128 + 4 * (8 * (r >> 2) + 4 * hf + (r & 3)) + s4;
        if (jj < Nk) wb[(int64_t)jj * p.EP + e] = acc[s4][r];
      }
  }
}

// Finalize: chain rule of the polar transform, both sides in one launch.
//   side 0 (blocks [0, nqb)): rows = queries of (b, h), acc = U, out = dq, phase row = q_off + i,
//                             no bias
//   side 1 (the rest):        rows = keys of (b, hk), acc = W, out = dk, phase row = j, dbias
//                             accumulated
// one workgroup = 32 rows of one (b, head); thread -> (4-dim quad, row group of 16), so that every
// load and store of the pass moves 16 bytes per lane (29.1 -> 22.3 us at C2 against one float per
// lane: the pass is bound by its loads in flight, not by its arithmetic).  The phases come from the
// tables when present, else are computed in place (sim_phase).
__global__ __launch_bounds__(kThreads) void sim_bwd_finalize_kernel(SimParams p, const float* U, const float* U2,
                                                                     const float* W, const float* W2, int nqb) {
  __shared__ float red[16][64];
  const int tid = threadIdx.x;
  const int side = (int)blockIdx.x < nqb ? 0 : 1;
  const float* acc = side == 0 ? U : W;
  const float* acc2 = side == 0 ? U2 : W2;
  const int nrb = side == 0 ? (p.Nq + 31) / 32 : (p.Nk + 31) / 32;
  const int blk = side == 0 ? (int)blockIdx.x : (int)blockIdx.x - nqb;
  const int rb = blk % nrb, bh = blk / nrb;
  const int heads = side == 0 ? p.Hq : p.Hk;
  const int b = bh / heads, hh = bh % heads;
  const int R = p.R, D = p.D, EP = p.EP;
  const int rows = side == 0 ? p.Nq : p.Nk;
  const int q_off = p.Nk - p.Nq;
  const float* x = side == 0 ? p.q + (int64_t)b * p.q_s[0] + (int64_t)hh * p.q_s[1]
                             : p.k + (int64_t)b * p.k_s[0] + (int64_t)hh * p.k_s[1];
  const int64_t xs = side == 0 ? p.q_s[2] : p.k_s[2];
  float* out = side == 0 ? p.dq + (int64_t)b * p.dq_s[0] + (int64_t)hh * p.dq_s[1]
                         : p.dk + (int64_t)b * p.dk_s[0] + (int64_t)hh * p.dk_s[1];
  const int64_t os = side == 0 ? p.dq_s[2] : p.dk_s[2];
  const float2* tab = nullptr;
  if (R && (side == 0 ? p.qtab : p.ktab))
    tab = side == 0 ? p.qtab + (int64_t)b * p.qt_sb + (int64_t)hh * p.qt_sh
                    : p.ktab + (int64_t)b * p.kt_sb + (int64_t)hh * p.kt_sh;
  const float* ab = acc + (int64_t)bh * rows * EP;
  // a second partial sum (split reduction of the split-bf16 path), added when present
  const float* ab2 = acc2 ? acc2 + (int64_t)bh * rows * EP : nullptr;
  float* part = side == 0 ? p.qpart : p.kpart;   // deterministic mode: written once, summed later
  // thread = (4-dim quad dq4 of a 64-dim chunk, row group rg of 16); every load and store moves 16 bytes
  const int dq4 = tid & 15, rg = tid >> 4;
  auto ld4 = [](const float* a) { return *reinterpret_cast<const float4*>(a); };
  // U / W rows are read once and dq / dk written once: non-temporal loads and stores (at C2 the
  // step ran about 4 us faster: 248.8 -> 244.5 us)
  auto ldnt = [](const float* a) {
    return __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a)));
  };

  for (int d0 = 0; d0 < D; d0 += 64) {
    const int d = d0 + 4 * dq4;
    float4 dps = make_float4(0.f, 0.f, 0.f, 0.f);
    if (d < D) {
      for (int rr = rg; rr < 32; rr += 16) {
        const int n = rb * 32 + rr;
        if (n >= rows) continue;
        const float* arow = ab + (int64_t)n * EP;
        const float* arow2 = ab2 ? ab2 + (int64_t)n * EP : nullptr;
        float* orow = out + (int64_t)n * os + d;
        if (d < R) {   // R is a multiple of 8: a quad is all rotated or all pass-through
          const int prow = side == 0 ? q_off + n : n;
          float cs[4], sn[4];
          if (tab) {
            const float4 t0 = ld4(reinterpret_cast<const float*>(tab + (int64_t)prow * R + d));
            const float4 t1 = ld4(reinterpret_cast<const float*>(tab + (int64_t)prow * R + d + 2));
            cs[0] = t0.x; sn[0] = t0.y; cs[1] = t0.z; sn[1] = t0.w;
            cs[2] = t1.x; sn[2] = t1.y; cs[3] = t1.z; sn[3] = t1.w;
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const float2 c2 = sim_phase(p, side, b, hh, prow, d + t);
              cs[t] = c2.x; sn[t] = c2.y;
            }
          }
          const float4 xv = ld4(x + (int64_t)n * xs + d);
          float4 uc = ldnt(arow + d), us = ldnt(arow + R + d);
          if (arow2) {
            const float4 uc2 = ldnt(arow2 + d), us2 = ldnt(arow2 + R + d);
            uc.x += uc2.x; uc.y += uc2.y; uc.z += uc2.z; uc.w += uc2.w;
            us.x += us2.x; us.y += us2.y; us.z += us2.z; us.w += us2.w;
          }
          const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
          const float ca[4] = {uc.x, uc.y, uc.z, uc.w}, sa[4] = {us.x, us.y, us.z, us.w};
          float g[4], dph[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            g[t] = sigmoid_f(xa[t]) * (cs[t] * ca[t] + sn[t] * sa[t]);
            dph[t] = softplus_f(xa[t]) * (cs[t] * sa[t] - sn[t] * ca[t]);
          }
          __builtin_nontemporal_store(f32x4{g[0], g[1], g[2], g[3]}, reinterpret_cast<f32x4*>(orow));
          if (part) {
            *reinterpret_cast<float4*>(part + ((int64_t)bh * rows + n) * R + d) = make_float4(dph[0], dph[1], dph[2], dph[3]);
          } else if (p.dfreqs) {
            float* df = p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)hh * p.df_s[1] + (int64_t)prow * p.df_s[2] + d;
#pragma unroll
            for (int t = 0; t < 4; ++t) atomicAdd(df + t, dph[t]);
          }
          dps.x += dph[0]; dps.y += dph[1]; dps.z += dph[2]; dps.w += dph[3];
        } else {
          float4 v = ldnt(arow + R + d);
          if (arow2) {
            const float4 v2 = ldnt(arow2 + R + d);
            v.x += v2.x; v.y += v2.y; v.z += v2.z; v.w += v2.w;
          }
          __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4*>(orow));
        }
      }
    }
    if (side == 1 && p.dbias && !p.kpart) {
      red[rg][4 * dq4] = dps.x; red[rg][4 * dq4 + 1] = dps.y; red[rg][4 * dq4 + 2] = dps.z; red[rg][4 * dq4 + 3] = dps.w;
      __syncthreads();
      if (tid < 64 && d0 + tid < R) {
        float s = 0.f;
#pragma unroll
        for (int g2 = 0; g2 < 16; ++g2) s += red[g2][tid];
        atomicAdd(p.dbias + (int64_t)hh * p.bias_sh + d0 + tid, s);
      }
      __syncthreads();
    }
  }
}

}  // namespace

hipError_t launch_sim_fwd(const SimParams& p, hipStream_t s) {
  const int nib = (p.Nq + 127) / 128, njb = (p.Nk + 127) / 128;
  const int blocks = nib * njb * p.B * p.Hq;
  return launch_named("sim_fwd", sim_fwd_kernel, dim3(blocks), dim3(kThreads), s, p, nib, njb);
}

// Workspace for U and W follows the two tables; the ABI passes it through SimParams::dsim-adjacent
// pointers set by the caller (see launch_sim_bwd_ws).
hipError_t launch_sim_bwd_ws(const SimParams& p, float* U, float* W, hipStream_t s) {
  const int nec = (p.EP + 127) / 128;
  const int nib = (p.Nq + 127) / 128, njb = (p.Nk + 127) / 128;
  hipError_t e = launch_named("sim_bwd_u", sim_bwd_u_kernel, dim3(nib * nec * p.B * p.Hq), dim3(kThreads), s, p, U,
                              nib, nec);
  if (e != hipSuccess) return e;
  e = launch_named("sim_bwd_w", sim_bwd_w_kernel, dim3(njb * nec * p.B * p.Hk), dim3(kThreads), s, p, W, njb, nec);
  if (e != hipSuccess) return e;
  return launch_sim_finalize(p, U, nullptr, W, nullptr, s);
}

hipError_t launch_sim_finalize(const SimParams& p, const float* U, const float* U2, const float* W, const float* W2,
                               hipStream_t s) {
  const int nrq = (p.Nq + 31) / 32, nrk = (p.Nk + 31) / 32;
  const int nqb = nrq * p.B * p.Hq;
  return launch_named("sim_bwd_finalize", sim_bwd_finalize_kernel, dim3(nqb + nrk * p.B * p.Hk), dim3(kThreads), s,
                      p, U, U2, W, W2, nqb);
}

}  // namespace pope
