// Flash attention backward with PoPE fused in (bf16 / fp16 MFMA, gfx950).
//
// Reference semantics: triton_pope_flash_attn.py:119-130 (_bwd_preprocess),
// :132-218 (_bwd_kernel) and :273-335 (launcher); PyTorch path
// attention.py:106-145 differentiated by autograd.
//
// With the expanded operands Q_hat (Nq x E) and K_hat (Nk x E) of
// pope_common.hpp and G = dL/dS = scale * P o (dO V^T - delta):
//   dV     = P^T dO
//   dK_hat = G^T Q_hat      dQ_hat = G K_hat
// and the chain rule of the polar transform (bias on the query side, as in the
// forward: query phase phi' = F[q_off + i] - bias, key phase psi = F[j]):
//   dq   = sigmoid(q) (cos phi' dQ_c + sin phi' dQ_s),  dq_rest = dQ_rest
//   dphi = softplus(q) (cos phi' dQ_s - sin phi' dQ_c)             -> dfreqs[q_off + i]
//   dk   = sigmoid(k) (cos psi dK_c + sin psi dK_s),    dk_rest = dK_rest
//   dpsi = softplus(k) (cos psi dK_s - sin psi dK_c)                -> dfreqs[j], dbias
// dbias = sum_j dpsi: S depends on phi' - psi only, so the derivative by the
// bias equals the summed key-phase derivative (the reference adds the same
// quantity, tl.sum(dfk, 0), triton_pope_flash_attn.py:210).
//
// Kernels (all on the caller's stream, no atomics except dfreqs / dbias):
//   prep_q : Q_hat rows and Q_hat^T, dO^T, delta = rowsum(O * dO) in fp32
//   prep_k : K_hat rows and K_hat^T
//   dkdv   : one workgroup = 128 keys (32 per wave) of one (batch, kv head);
//            loops over the query heads of its group and the query tiles that
//            can see its keys (causal tiles before the diagonal are skipped);
//            epilogue applies the key-side chain rule and sums dbias.
//   dq     : one workgroup = 128 queries (32 per wave); loops over the key
//            tiles up to the causal diagonal; epilogue applies the query-side
//            chain rule.  dQ needs no atomics, so the result is deterministic
//            (the reference accumulates dq with atomics in the input dtype,
//            triton_pope_flash_attn.py:215).
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(uint16_t* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

// B/A operand of 8 elements gathered as two runs of 4: [p, p+4) and [p+8, p+12).
// This is the k-slot order of a 16-wide group of a 32x32 MFMA result read back
// as an operand (result rows 8*(r/4) + 4*half + r%4).
__device__ __forceinline__ u32x4 ld_split8(const uint16_t* p) {
  const u32x2 lo = *reinterpret_cast<const u32x2*>(p);
  const u32x2 hi = *reinterpret_cast<const u32x2*>(p + 8);
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* x) {
  u32x4 w;
#pragma unroll
  for (int s = 0; s < 4; ++s) w[s] = T::pack2(x[2 * s], x[2 * s + 1]);
  return w;
}

// Registers [8 g, 8 g + 8) of an MFMA result, packed as an 8-element operand.
template <typename T>
__device__ __forceinline__ u32x4 pack8(const f32x16& x, int g) {
  u32x4 w;
#pragma unroll
  for (int s = 0; s < 4; ++s) w[s] = T::pack2(x[8 * g + 2 * s], x[8 * g + 2 * s + 1]);
  return w;
}

// ---------------------------------------------------------------------------
// prep_q: one thread per (batch, query head, padded query row).
template <typename T>
__global__ __launch_bounds__(kThreads) void bwd_prep_q_kernel(FlashBwdParams p) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= (int64_t)p.B * p.Hq * p.NqP) return;
  const int i = (int)(idx % p.NqP);
  const int bh = (int)(idx / p.NqP);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int D = p.D, R = p.R, E = p.E, EP = p.EP, NqP = p.NqP;
  const bool valid = i < p.Nq;
  const int q_off = p.Nk - p.Nq;

  const uint16_t* qrow = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1] + (int64_t)i * p.q_s[2];
  const float* frow = R ? p.freqs + (int64_t)b * p.f_s[0] + (int64_t)h * p.f_s[1] + (int64_t)(q_off + i) * p.f_s[2]
                        : nullptr;
  const float* brow = R ? p.bias + (int64_t)hk * p.bias_sh : nullptr;
  uint16_t* qh_row = p.qh + ((int64_t)bh * NqP + i) * EP;
  uint16_t* qht_col = p.qht + (int64_t)bh * EP * NqP + i;
  for (int e0 = 0; e0 < EP; e0 += 8) {
    float out[8];
    if (!valid || e0 >= E) {
#pragma unroll
      for (int s = 0; s < 8; ++s) out[s] = 0.f;
    } else {
      const bool is_cos = e0 < R, is_sin = !is_cos && e0 < 2 * R;
      const int d0 = is_cos ? e0 : e0 - R;
      float x[8];
      unpack8<T>(ld16(qrow + d0), x);
      if (is_cos || is_sin) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          float sn, cs;
          sincos_acc(frow[d0 + s] - brow[d0 + s], &sn, &cs);
          out[s] = softplus_f(x[s]) * (is_cos ? cs : sn);
        }
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) out[s] = x[s];
      }
    }
    const u32x4 w = pack8<T>(out);
    st16(qh_row + e0, w);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qht_col[(int64_t)(e0 + 2 * s) * NqP] = (uint16_t)u16lo(w[s]);
      qht_col[(int64_t)(e0 + 2 * s + 1) * NqP] = (uint16_t)u16hi(w[s]);
    }
  }

  const uint16_t* orow = p.o + (int64_t)b * p.o_s[0] + (int64_t)h * p.o_s[1] + (int64_t)i * p.o_s[2];
  const uint16_t* drow = p.dout + (int64_t)b * p.do_s[0] + (int64_t)h * p.do_s[1] + (int64_t)i * p.do_s[2];
  uint16_t* dot_col = p.dot + (int64_t)bh * p.DV * NqP + i;
  float dl = 0.f;
  for (int d0 = 0; d0 < p.DV; d0 += 8) {
    u32x4 wd = zero4();
    if (valid && d0 < D) {
      wd = ld16(drow + d0);
      float xo[8], xd[8];
      unpack8<T>(ld16(orow + d0), xo);
      unpack8<T>(wd, xd);
#pragma unroll
      for (int s = 0; s < 8; ++s) dl += xo[s] * xd[s];
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      dot_col[(int64_t)(d0 + 2 * s) * NqP] = (uint16_t)u16lo(wd[s]);
      dot_col[(int64_t)(d0 + 2 * s + 1) * NqP] = (uint16_t)u16hi(wd[s]);
    }
  }
  p.delta[(int64_t)bh * NqP + i] = dl;
}

// prep_k: one thread per (batch, kv head, padded key row).
template <typename T>
__global__ __launch_bounds__(kThreads) void bwd_prep_k_kernel(FlashBwdParams p) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= (int64_t)p.B * p.Hk * p.NkP) return;
  const int j = (int)(idx % p.NkP);
  const int bhk = (int)(idx / p.NkP);
  const int b = bhk / p.Hk, hk = bhk % p.Hk;
  const int R = p.R, E = p.E, EP = p.EP, NkP = p.NkP;
  const bool valid = j < p.Nk;
  const uint16_t* krow = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1] + (int64_t)j * p.k_s[2];
  const float2* trow = R ? p.table + (int64_t)b * p.t_sb + (int64_t)hk * p.t_sh + (int64_t)j * R : nullptr;
  uint16_t* kh_row = p.kh + ((int64_t)bhk * NkP + j) * EP;
  uint16_t* kht_col = p.kht + (int64_t)bhk * EP * NkP + j;
  for (int e0 = 0; e0 < EP; e0 += 8) {
    float out[8];
    if (!valid || e0 >= E) {
#pragma unroll
      for (int s = 0; s < 8; ++s) out[s] = 0.f;
    } else {
      const bool is_cos = e0 < R, is_sin = !is_cos && e0 < 2 * R;
      const int d0 = is_cos ? e0 : e0 - R;
      float x[8];
      unpack8<T>(ld16(krow + d0), x);
      if (is_cos || is_sin) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const float2 t = trow[d0 + s];
          out[s] = softplus_f(x[s]) * (is_cos ? t.x : t.y);
        }
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) out[s] = x[s];
      }
    }
    const u32x4 w = pack8<T>(out);
    st16(kh_row + e0, w);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      kht_col[(int64_t)(e0 + 2 * s) * NkP] = (uint16_t)u16lo(w[s]);
      kht_col[(int64_t)(e0 + 2 * s + 1) * NkP] = (uint16_t)u16hi(w[s]);
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV.  Lane roles: lane lr of wave w owns key j0 + 32 w + lr.
//   S  = Q_hat K_hat^T : A = Q_hat tile rows (LDS), B = the lane's K_hat row (regs)
//   dP = dO V^T        : A = dO tile rows (LDS),    B = the lane's V row (regs)
// Both results have lane = key, registers = queries, so P and dS feed the next
// products directly as A operands (lane = key row, k-slots = queries):
//   dV     += P^T dO      B = dO^T  tile (LDS, [d][query])
//   dK_hat += dS^T Q_hat  B = Q_hat^T tile (LDS, [e][query])
template <typename T, int EP, int DV, int BM, int MINB>
__global__ __launch_bounds__(kThreads, MINB) void bwd_dkdv_kernel(FlashBwdParams p) {
  constexpr int BN = 128;
  constexpr int KS = EP / 16, DS = DV / 16, EB = EP / 32, DB = DV / 32, QB = BM / 32;
  constexpr int QH = EP + 8, QT = BM + 8, DO = DV + 8;
  constexpr int MAIN = (BM * QH + EP * QT + BM * DO + DV * QT) * 2 + 2 * BM * 4;
  constexpr int BS = EP + 1;
  constexpr int EPI = 32 * BS * 4;
  constexpr int LDS = MAIN > EPI ? MAIN : EPI;
  typedef typename T::vec8 vec8;

  __shared__ __attribute__((aligned(16))) char smem[LDS];
  __shared__ float dbias_s[EP];
  uint16_t* qh_s = reinterpret_cast<uint16_t*>(smem);
  uint16_t* qht_s = qh_s + BM * QH;
  uint16_t* do_s = qht_s + EP * QT;
  uint16_t* dot_s = do_s + BM * DO;
  float* lse_s = reinterpret_cast<float*>(dot_s + DV * QT);
  float* dl_s = lse_s + BM;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int nkb = p.NkP / BN;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int kb = id % nkb, bhk = id / nkb;
  const int b = bhk / p.Hk, hk = bhk % p.Hk;
  const int D = p.D, R = p.R, Nq = p.Nq, Nk = p.Nk, NqP = p.NqP;
  const int j0 = kb * BN;
  const int kj = j0 + 32 * wave + lr;

  const uint8_t* mrow = p.has_mask ? p.mask + (int64_t)b * p.mask_sb : nullptr;
  const bool kvis = kj < Nk && (!p.has_mask || mrow[kj] != 0);

  for (int e = tid; e < EP; e += kThreads) dbias_s[e] = 0.f;

  // This lane's K_hat and V rows as B operands (k-slots 16 kk + 8 hf ...).
  vec8 kreg[KS], vreg[DS];
  {
    const uint16_t* khr = p.kh + ((int64_t)bhk * p.NkP + kj) * EP;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) kreg[kk] = as_vec8<vec8>(ld16(khr + 16 * kk + 8 * hf));
    const uint16_t* vr = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1] + (int64_t)min(kj, Nk - 1) * p.v_s[2];
#pragma unroll
    for (int kk = 0; kk < DS; ++kk) {
      const int d0 = 16 * kk + 8 * hf;
      vreg[kk] = as_vec8<vec8>((kj < Nk && d0 < D) ? ld16(vr + d0) : zero4());
    }
  }

  f32x16 dva[DB], dka[EB];
#pragma unroll
  for (int x = 0; x < DB; ++x)
#pragma unroll
    for (int r = 0; r < 16; ++r) dva[x][r] = 0.f;
#pragma unroll
  for (int x = 0; x < EB; ++x)
#pragma unroll
    for (int r = 0; r < 16; ++r) dka[x][r] = 0.f;

  const int any_key = __syncthreads_or(kvis ? 1 : 0);
  const int nqt = (Nq + BM - 1) / BM;
  const int qt0 = p.causal ? j0 / BM : 0;
  const int groups = p.Hq / p.Hk;

  if (any_key) {
    for (int g = 0; g < groups; ++g) {
      const int h = hk + g * p.Hk;
      const int bh = b * p.Hq + h;
      const uint16_t* qh_g = p.qh + (int64_t)bh * NqP * EP;
      const uint16_t* qht_g = p.qht + (int64_t)bh * EP * NqP;
      const uint16_t* dot_g = p.dot + (int64_t)bh * DV * NqP;
      const uint16_t* do_g = p.dout + (int64_t)b * p.do_s[0] + (int64_t)h * p.do_s[1];
      for (int qt = qt0; qt < nqt; ++qt) {
        const int i0 = qt * BM;
        __syncthreads();
        for (int c = tid; c < BM * (EP / 8); c += kThreads) {
          const int row = c / (EP / 8), c8 = c % (EP / 8);
          st16(qh_s + row * QH + 8 * c8, ld16(qh_g + (int64_t)(i0 + row) * EP + 8 * c8));
        }
        for (int c = tid; c < EP * (BM / 8); c += kThreads) {
          const int e = c / (BM / 8), c8 = c % (BM / 8);
          st16(qht_s + e * QT + 8 * c8, ld16(qht_g + (int64_t)e * NqP + i0 + 8 * c8));
        }
        for (int c = tid; c < BM * (DV / 8); c += kThreads) {
          const int row = c / (DV / 8), c8 = c % (DV / 8);
          u32x4 w = zero4();
          if (i0 + row < Nq && 8 * c8 < D) w = ld16(do_g + (int64_t)(i0 + row) * p.do_s[2] + 8 * c8);
          st16(do_s + row * DO + 8 * c8, w);
        }
        for (int c = tid; c < DV * (BM / 8); c += kThreads) {
          const int d = c / (BM / 8), c8 = c % (BM / 8);
          st16(dot_s + d * QT + 8 * c8, ld16(dot_g + (int64_t)d * NqP + i0 + 8 * c8));
        }
        if (tid < BM) {
          const int i = i0 + tid;
          const float l = i < Nq ? p.lse[(int64_t)bh * Nq + i] : -INFINITY;
          lse_s[tid] = l == -INFINITY ? INFINITY : l * kLog2e;
          dl_s[tid] = p.delta[(int64_t)bh * NqP + i];
        }
        __syncthreads();

#pragma unroll
        for (int qs = 0; qs < QB; ++qs) {
          f32x16 s, dp;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s[r] = 0.f;
            dp[r] = 0.f;
          }
#pragma unroll
          for (int kk = 0; kk < KS; ++kk) {
            const vec8 a = as_vec8<vec8>(ld16(qh_s + (32 * qs + lr) * QH + 16 * kk + 8 * hf));
            s = T::mfma32(a, kreg[kk], s);
          }
#pragma unroll
          for (int kk = 0; kk < DS; ++kk) {
            const vec8 a = as_vec8<vec8>(ld16(do_s + (32 * qs + lr) * DO + 16 * kk + 8 * hf));
            dp = T::mfma32(a, vreg[kk], dp);
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int qr = 32 * qs + 8 * (r >> 2) + 4 * hf + (r & 3);
            const bool vis = kvis && (!p.causal || kj <= i0 + qr);
            const float pv = vis ? __builtin_amdgcn_exp2f(fmaf(s[r], p.scale_log2, -lse_s[qr])) : 0.f;
            s[r] = pv;
            dp[r] = pv * (dp[r] - dl_s[qr]);
          }
#pragma unroll
          for (int g2 = 0; g2 < 2; ++g2) {
            const vec8 ap = as_vec8<vec8>(pack8<T>(s, g2));
            const vec8 ads = as_vec8<vec8>(pack8<T>(dp, g2));
            const int col = 32 * qs + 16 * g2 + 4 * hf;
#pragma unroll
            for (int db = 0; db < DB; ++db)
              dva[db] = T::mfma32(ap, as_vec8<vec8>(ld_split8(dot_s + (32 * db + lr) * QT + col)), dva[db]);
#pragma unroll
            for (int eb = 0; eb < EB; ++eb)
              dka[eb] = T::mfma32(ads, as_vec8<vec8>(ld_split8(qht_s + (32 * eb + lr) * QT + col)), dka[eb]);
          }
        }
      }
    }
  }

  // ---- dV: lane = d column, registers = the wave's keys -----------------------
  {
    uint16_t* dvb = p.dv + (int64_t)b * p.dv_s[0] + (int64_t)hk * p.dv_s[1];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int d = 32 * db + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = j0 + 32 * wave + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (key < Nk && d < D) dvb[(int64_t)key * p.dv_s[2] + d] = T::bits(dva[db][r]);
      }
    }
  }

  // ---- dK: key-side chain rule, one wave's 32 keys at a time through LDS -------
  float* buf = reinterpret_cast<float*>(smem);
  const uint16_t* kb_ptr = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1];
  uint16_t* dkb = p.dk + (int64_t)b * p.dk_s[0] + (int64_t)hk * p.dk_s[1];
  const float2* tb = R ? p.table + (int64_t)b * p.t_sb + (int64_t)hk * p.t_sh : nullptr;
  float* dfb = p.dfreqs ? p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)hk * p.df_s[1] : nullptr;
  for (int w = 0; w < 4; ++w) {
    __syncthreads();
    if (wave == w) {
#pragma unroll
      for (int eb = 0; eb < EB; ++eb)
#pragma unroll
        for (int r = 0; r < 16; ++r) buf[(8 * (r >> 2) + 4 * hf + (r & 3)) * BS + 32 * eb + lr] = dka[eb][r];
    }
    __syncthreads();
    for (int it = tid; it < 32 * D; it += kThreads) {
      const int kr = it / D, d = it - kr * D;
      const int key = j0 + 32 * w + kr;
      if (key >= Nk) continue;
      const float* row = buf + kr * BS;
      float g;
      if (d < R) {
        const float x = T::to_float(kb_ptr[(int64_t)key * p.k_s[2] + d]);
        const float2 cs = tb[(int64_t)key * R + d];
        const float uc = row[d] * p.scale, us = row[R + d] * p.scale;
        g = sigmoid_f(x) * (cs.x * uc + cs.y * us);
        const float dpsi = softplus_f(x) * (cs.x * us - cs.y * uc);
        if (dfb) atomicAdd(dfb + (int64_t)key * p.df_s[2] + d, dpsi);
        if (p.dbias) atomicAdd(&dbias_s[d], dpsi);
      } else {
        g = row[R + d] * p.scale;
      }
      dkb[(int64_t)key * p.dk_s[2] + d] = T::bits(g);
    }
  }
  if (p.dbias) {
    __syncthreads();
    for (int d = tid; d < R; d += kThreads) atomicAdd(p.dbias + (int64_t)hk * p.bias_sh + d, dbias_s[d]);
  }
}

// ---------------------------------------------------------------------------
// dQ.  Lane roles: lane lr of wave w owns query i0 + 32 w + lr.
//   S^T  = K_hat Q_hat^T : A = K_hat tile rows (LDS), B = the lane's Q_hat row (regs)
//   dP^T = V dO^T        : A = V tile rows (LDS),     B = the lane's dO row (regs)
// Results: lane = query, registers = keys; dS^T feeds dQ_hat^T = K_hat^T dS^T
// as the B operand, with A = K_hat^T tile (LDS, [e][key]).
template <typename T, int EP, int DV, int BN, int MINB>
__global__ __launch_bounds__(kThreads, MINB) void bwd_dq_kernel(FlashBwdParams p) {
  constexpr int BM = 128;
  constexpr int KS = EP / 16, DS = DV / 16, EB = EP / 32, NB = BN / 32;
  constexpr int KH = EP + 8, KT = BN + 8, VR = DV + 8;
  constexpr int MAIN = (BN * KH + EP * KT + BN * VR) * 2;
  constexpr int BS = EP + 1;
  constexpr int EPI = 32 * BS * 4;
  constexpr int LDS = MAIN > EPI ? MAIN : EPI;
  typedef typename T::vec8 vec8;

  __shared__ __attribute__((aligned(16))) char smem[LDS];
  __shared__ uint8_t msk_s[BN];
  uint16_t* kh_s = reinterpret_cast<uint16_t*>(smem);
  uint16_t* kht_s = kh_s + BN * KH;
  uint16_t* v_s = kht_s + EP * KT;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int nqb = p.NqP / BM;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int qb = nqb - 1 - (id % nqb), bh = id / nqb;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int bhk = b * p.Hk + hk;
  const int D = p.D, R = p.R, Nq = p.Nq, Nk = p.Nk, NkP = p.NkP;
  const int q_off = Nk - Nq;
  const int qi = qb * BM + 32 * wave + lr;
  const bool qvalid = qi < Nq;

  vec8 qreg[KS], doreg[DS];
  {
    const uint16_t* qhr = p.qh + ((int64_t)bh * p.NqP + qi) * EP;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qreg[kk] = as_vec8<vec8>(ld16(qhr + 16 * kk + 8 * hf));
    const uint16_t* dr = p.dout + (int64_t)b * p.do_s[0] + (int64_t)h * p.do_s[1] +
                         (int64_t)min(qi, Nq - 1) * p.do_s[2];
#pragma unroll
    for (int kk = 0; kk < DS; ++kk) {
      const int d0 = 16 * kk + 8 * hf;
      doreg[kk] = as_vec8<vec8>((qvalid && d0 < D) ? ld16(dr + d0) : zero4());
    }
  }
  float lse2 = INFINITY, dl = 0.f;
  if (qvalid) {
    const float l = p.lse[(int64_t)bh * Nq + qi];
    lse2 = l == -INFINITY ? INFINITY : l * kLog2e;
    dl = p.delta[(int64_t)bh * p.NqP + qi];
  }

  f32x16 dqa[EB];
#pragma unroll
  for (int x = 0; x < EB; ++x)
#pragma unroll
    for (int r = 0; r < 16; ++r) dqa[x][r] = 0.f;

  int kt_end = (Nk + BN - 1) / BN;
  if (p.causal) {
    const int last_q = min(qb * BM + BM, Nq) - 1;
    kt_end = last_q < 0 ? 0 : min(kt_end, last_q / BN + 1);
  }
  const uint16_t* kh_g = p.kh + (int64_t)bhk * NkP * EP;
  const uint16_t* kht_g = p.kht + (int64_t)bhk * EP * NkP;
  const uint16_t* v_g = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  const uint8_t* mrow = p.has_mask ? p.mask + (int64_t)b * p.mask_sb : nullptr;

  for (int kt = 0; kt < kt_end; ++kt) {
    const int j0 = kt * BN;
    __syncthreads();
    for (int c = tid; c < BN * (EP / 8); c += kThreads) {
      const int row = c / (EP / 8), c8 = c % (EP / 8);
      st16(kh_s + row * KH + 8 * c8, ld16(kh_g + (int64_t)(j0 + row) * EP + 8 * c8));
    }
    for (int c = tid; c < EP * (BN / 8); c += kThreads) {
      const int e = c / (BN / 8), c8 = c % (BN / 8);
      st16(kht_s + e * KT + 8 * c8, ld16(kht_g + (int64_t)e * NkP + j0 + 8 * c8));
    }
    for (int c = tid; c < BN * (DV / 8); c += kThreads) {
      const int row = c / (DV / 8), c8 = c % (DV / 8);
      u32x4 w = zero4();
      if (j0 + row < Nk && 8 * c8 < D) w = ld16(v_g + (int64_t)(j0 + row) * p.v_s[2] + 8 * c8);
      st16(v_s + row * VR + 8 * c8, w);
    }
    int vis = 0;
    if (tid < BN) {
      const int key = j0 + tid;
      vis = key < Nk && (!p.has_mask || mrow[key] != 0);
      msk_s[tid] = (uint8_t)vis;
    }
    if (!__syncthreads_or(vis)) continue;   // every key of this tile masked

#pragma unroll
    for (int ks = 0; ks < NB; ++ks) {
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = 0.f;
        dp[r] = 0.f;
      }
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const vec8 a = as_vec8<vec8>(ld16(kh_s + (32 * ks + lr) * KH + 16 * kk + 8 * hf));
        s = T::mfma32(a, qreg[kk], s);
      }
#pragma unroll
      for (int kk = 0; kk < DS; ++kk) {
        const vec8 a = as_vec8<vec8>(ld16(v_s + (32 * ks + lr) * VR + 16 * kk + 8 * hf));
        dp = T::mfma32(a, doreg[kk], dp);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 32 * ks + 8 * (r >> 2) + 4 * hf + (r & 3);
        const bool ok = msk_s[kr] && (!p.causal || j0 + kr <= qi);
        const float pv = ok ? __builtin_amdgcn_exp2f(fmaf(s[r], p.scale_log2, -lse2)) : 0.f;
        dp[r] = pv * (dp[r] - dl);
      }
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const vec8 bds = as_vec8<vec8>(pack8<T>(dp, g2));
        const int col = 32 * ks + 16 * g2 + 4 * hf;
#pragma unroll
        for (int eb = 0; eb < EB; ++eb)
          dqa[eb] = T::mfma32(as_vec8<vec8>(ld_split8(kht_s + (32 * eb + lr) * KT + col)), bds, dqa[eb]);
      }
    }
  }

  // ---- dQ: query-side chain rule, one wave's 32 queries at a time through LDS ----
  float* buf = reinterpret_cast<float*>(smem);
  const uint16_t* qb_ptr = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1];
  uint16_t* dqb = p.dq + (int64_t)b * p.dq_s[0] + (int64_t)h * p.dq_s[1];
  const float* fb = R ? p.freqs + (int64_t)b * p.f_s[0] + (int64_t)h * p.f_s[1] : nullptr;
  const float* brow = R ? p.bias + (int64_t)hk * p.bias_sh : nullptr;
  float* dfb = p.dfreqs ? p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)h * p.df_s[1] : nullptr;
  for (int w = 0; w < 4; ++w) {
    __syncthreads();
    if (wave == w) {
#pragma unroll
      for (int eb = 0; eb < EB; ++eb)
#pragma unroll
        for (int r = 0; r < 16; ++r) buf[lr * BS + 32 * eb + 8 * (r >> 2) + 4 * hf + (r & 3)] = dqa[eb][r];
    }
    __syncthreads();
    for (int it = tid; it < 32 * D; it += kThreads) {
      const int qr = it / D, d = it - qr * D;
      const int i = qb * BM + 32 * w + qr;
      if (i >= Nq) continue;
      const float* row = buf + qr * BS;
      float g;
      if (d < R) {
        const float x = T::to_float(qb_ptr[(int64_t)i * p.q_s[2] + d]);
        float sn, cs;
        sincos_acc(fb[(int64_t)(q_off + i) * p.f_s[2] + d] - brow[d], &sn, &cs);
        const float uc = row[d] * p.scale, us = row[R + d] * p.scale;
        g = sigmoid_f(x) * (cs * uc + sn * us);
        if (dfb) atomicAdd(dfb + (int64_t)(q_off + i) * p.df_s[2] + d, softplus_f(x) * (cs * us - sn * uc));
      } else {
        g = row[R + d] * p.scale;
      }
      dqb[(int64_t)i * p.dq_s[2] + d] = T::bits(g);
    }
  }
}

template <typename T, int EP, int DV>
hipError_t launch_t(const FlashBwdParams& p, hipStream_t s) {
  constexpr bool kBig = EP + DV > 160;
  constexpr int BMK = kBig ? 32 : 64;   // query tile of the dK/dV kernel
  constexpr int BNQ = kBig ? 32 : 64;   // key tile of the dQ kernel
  constexpr int MINB = kBig ? 1 : 2;
  const int64_t nq = (int64_t)p.B * p.Hq * p.NqP, nk = (int64_t)p.B * p.Hk * p.NkP;
  hipError_t e = launch_named("flash_bwd_prep_q", bwd_prep_q_kernel<T>,
                              dim3((unsigned)((nq + kThreads - 1) / kThreads)), dim3(kThreads), s, p);
  if (e != hipSuccess) return e;
  e = launch_named("flash_bwd_prep_k", bwd_prep_k_kernel<T>, dim3((unsigned)((nk + kThreads - 1) / kThreads)),
                   dim3(kThreads), s, p);
  if (e != hipSuccess) return e;
  e = launch_named("flash_bwd_dkdv", bwd_dkdv_kernel<T, EP, DV, BMK, MINB>, dim3((p.NkP / 128) * p.B * p.Hk),
                   dim3(kThreads), s, p);
  if (e != hipSuccess) return e;
  return launch_named("flash_bwd_dq", bwd_dq_kernel<T, EP, DV, BNQ, MINB>, dim3((p.NqP / 128) * p.B * p.Hq),
                      dim3(kThreads), s, p);
}

template <typename T>
hipError_t dispatch(const FlashBwdParams& p, hipStream_t s) {
#define POPE_BWD_CASE(ep, dv) \
  if (p.EP == ep && p.DV == dv) return launch_t<T, ep, dv>(p, s);
  POPE_BWD_CASE(32, 32) POPE_BWD_CASE(64, 32)
  POPE_BWD_CASE(64, 64) POPE_BWD_CASE(96, 64) POPE_BWD_CASE(128, 64)
  POPE_BWD_CASE(96, 96) POPE_BWD_CASE(128, 96) POPE_BWD_CASE(160, 96) POPE_BWD_CASE(192, 96)
  POPE_BWD_CASE(128, 128) POPE_BWD_CASE(160, 128) POPE_BWD_CASE(192, 128) POPE_BWD_CASE(224, 128)
  POPE_BWD_CASE(256, 128)
#undef POPE_BWD_CASE
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_flash_bwd(const FlashBwdParams& p, int dtype, hipStream_t s) {
  return dtype == 2 ? dispatch<BF16>(p, s) : dispatch<F16>(p, s);
}

}  // namespace pope
