// Flash attention forward with PoPE fused in (bf16 / fp16 MFMA, gfx950).
//
// Reference semantics: triton_pope_flash_attn.py:23-117 (kernel) and :222-271
// (launcher); PyTorch path attention.py:106-145.
//
// Work decomposition
//   one workgroup = 4 waves = 128 query rows of one (batch, query head);
//   each wave owns 32 query rows; the key axis is swept in tiles of BN = 64.
// Per key tile
//   K is loaded, put through the polar transform and written to LDS as
//   K_hat[key][e] (E = D + R expanded columns, see pope_common.hpp);
//   V is written to LDS transposed, Vt[d][key].
//   S^T = K_hat Q_hat^T runs on v_mfma_f32_32x32x16 with K_hat as the A operand
//   (lane = key) and the wave's Q_hat, held in registers for the whole sweep,
//   as the B operand (lane = query).  The result puts one query per lane and
//   keys in registers, so the softmax row reductions stay in-lane (plus one
//   swap between the two lane halves).
//   O^T += Vt P^T reuses the probabilities straight from the S registers as
//   the B operand (a key permutation inside each 16-key group that the Vt
//   reads follow).
// Phases
//   The learned bias is moved to the query side: cos(phi - (F_j + b)) =
//   cos((phi - b) - F_j), so Q_hat = a * (cos, sin)(F[q_off+i] - b) is computed
//   once per workgroup with accurate sincos and K_hat = c * (cos, sin)(F_j)
//   reads the per-call table of cos/sin(F).  Differences to the reference's
//   fl(F_j + b) rounding are below bf16 resolution.
// Masking
//   top-left causal (key j visible to query i iff j <= i, the SDPA convention
//   the reference uses, triton_pope_flash_attn.py:64,86-87), key padding mask
//   (nonzero = keep), keys >= Nk.  Key tiles past the causal diagonal are never
//   visited; a tile that leaves every row of a wave masked is skipped.  Fully
//   masked rows give O = 0 and LSE = -inf (:114,117).
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kFwdBM = 128;
constexpr int kFwdBN = 64;
constexpr int kFwdThreads = 256;

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

template <typename T, int EP, int DV>
__global__ __launch_bounds__(kFwdThreads, 2) void flash_fwd_kernel(FlashFwdParams p) {
  constexpr int BN = kFwdBN;
  constexpr int KSTEPS = EP / 16;
  constexpr int KH = EP + 8;   // K_hat row stride (elements); +8 spreads rows over LDS banks
  constexpr int VT = BN + 4;   // Vt row stride (elements)
  constexpr int NDB = DV / 32;
  typedef typename T::vec8 vec8;

  __shared__ __attribute__((aligned(16))) uint16_t kh[BN * KH];
  __shared__ __attribute__((aligned(16))) uint16_t vt[DV * VT];
  __shared__ uint32_t mskw[BN / 4];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = id / p.nqb;
  const int qb = p.nqb - 1 - (id % p.nqb);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int D = p.D, R = p.R, E = D + R, Nk = p.Nk, Nq = p.Nq;
  const int q_off = Nk - Nq;
  const int qi = qb * kFwdBM + wave * 32 + lr;
  const bool qvalid = qi < Nq;

  // Zero the padding that the tile loops never write.
  for (int i = tid; i < BN * (EP - E); i += kFwdThreads) {
    int j = i / (EP - E), c = i % (EP - E);
    kh[j * KH + E + c] = 0;
  }
  for (int i = tid; i < (DV - D) * VT; i += kFwdThreads) vt[D * VT + i] = 0;

  // ---- Q_hat for this lane's query row, in MFMA B-operand order ----------
  vec8 qreg[KSTEPS];
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1] + (int64_t)qi * p.q_s[2];
    const float* frow = p.freqs ? p.freqs + (int64_t)b * p.f_s[0] + (int64_t)h * p.f_s[1] +
                                      (int64_t)(q_off + qi) * p.f_s[2]
                                : nullptr;
    const float* brow = p.bias ? p.bias + (int64_t)hk * p.bias_sh : nullptr;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const int e0 = 16 * kk + 8 * hf;
      float out[8];
      if (!qvalid || e0 >= E) {
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
      u32x4 w;
#pragma unroll
      for (int s = 0; s < 4; ++s) w[s] = T::pack2(out[2 * s], out[2 * s + 1]);
      qreg[kk] = as_vec8<vec8>(w);
    }
  }

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  int kt_end = (Nk + BN - 1) / BN;
  if (p.causal) {
    const int last_q = min(qb * kFwdBM + kFwdBM, Nq) - 1;
    kt_end = min(kt_end, last_q / BN + 1);
  }
  const int nch = D / 8;
  const uint16_t* kbase = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1];
  const uint16_t* vbase = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  const float2* tbase = p.table ? p.table + (int64_t)b * p.t_sb + (int64_t)h * p.t_sh : nullptr;

  for (int kt = 0; kt < kt_end; ++kt) {
    const int j0 = kt * BN;
    __syncthreads();
    // ---- K tile -> K_hat in LDS ------------------------------------------
    for (int it = tid; it < BN * nch; it += kFwdThreads) {
      const int j = it / nch, c = it - j * nch, key = j0 + j, d0 = c * 8;
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (key < Nk) raw = ld16(kbase + (int64_t)key * p.k_s[2] + d0);
      if (d0 < R) {
        float x[8];
        unpack8<T>(raw, x);
        const float4* tp = reinterpret_cast<const float4*>(tbase + (int64_t)min(key, Nk - 1) * R + d0);
        u32x4 wc, ws;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float4 t = tp[s];  // (cos, sin) of dims d0+2s, d0+2s+1
          float a0 = softplus_f(x[2 * s]), a1 = softplus_f(x[2 * s + 1]);
          wc[s] = T::pack2(a0 * t.x, a1 * t.z);
          ws[s] = T::pack2(a0 * t.y, a1 * t.w);
        }
        *reinterpret_cast<u32x4*>(&kh[j * KH + d0]) = wc;
        *reinterpret_cast<u32x4*>(&kh[j * KH + R + d0]) = ws;
      } else {
        *reinterpret_cast<u32x4*>(&kh[j * KH + R + d0]) = raw;
      }
    }
    // ---- V tile -> Vt in LDS (key pairs packed per 32-bit word) ------------
    for (int it = tid; it < (BN / 2) * nch; it += kFwdThreads) {
      const int pr = it / nch, c = it - pr * nch, key = j0 + 2 * pr, d0 = c * 8;
      u32x4 r0 = {0u, 0u, 0u, 0u}, r1 = {0u, 0u, 0u, 0u};
      if (key < Nk) r0 = ld16(vbase + (int64_t)key * p.v_s[2] + d0);
      if (key + 1 < Nk) r1 = ld16(vbase + (int64_t)(key + 1) * p.v_s[2] + d0);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        *reinterpret_cast<uint32_t*>(&vt[(d0 + 2 * s) * VT + 2 * pr]) = u16lo(r0[s]) | (u16lo(r1[s]) << 16);
        *reinterpret_cast<uint32_t*>(&vt[(d0 + 2 * s + 1) * VT + 2 * pr]) = u16hi(r0[s]) | (u16hi(r1[s]) << 16);
      }
    }
    if (tid < BN / 4) {
      uint32_t w = 0;
      if (p.has_mask) {
        const uint8_t* mrow = p.mask + (int64_t)b * p.mask_sb;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int key = j0 + 4 * tid + s;
          w |= (key < Nk && mrow[key]) ? (1u << (8 * s)) : 0u;
        }
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) w |= (j0 + 4 * tid + s < Nk) ? (1u << (8 * s)) : 0u;
      }
      mskw[tid] = w;
    }
    __syncthreads();

    // ---- S^T = K_hat Q_hat^T ---------------------------------------------
    f32x16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        vec8 a = as_vec8<vec8>(*reinterpret_cast<const u32x4*>(&kh[(32 * kb + lr) * KH + 16 * kk + 8 * hf]));
        sacc[kb] = T::mfma32(a, qreg[kk], sacc[kb]);
      }
    }
    // ---- scale + masks + running max --------------------------------------
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t mw = mskw[8 * kb + 2 * g + hf];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * g + i;
          const int key = j0 + 32 * kb + 8 * g + 4 * hf + i;
          const bool ok = ((mw >> (8 * i)) & 0xffu) && (!p.causal || key <= qi);
          const float s = ok ? sacc[kb][r] * p.scale_log2 : -INFINITY;
          sacc[kb][r] = s;
          mt = fmaxf(mt, s);
        }
      }
    }
    mt = fmaxf(mt, wave_shfl_xor(mt, 32));
    if (!__any(mt > -INFINITY)) continue;  // every row of this wave masked for this tile
    const float m_new = fmaxf(m_run, mt);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = __builtin_amdgcn_exp2f(sacc[kb][r] - m_use);
        sacc[kb][r] = pr;
        psum += pr;
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;

    // ---- O^T += Vt P^T ---------------------------------------------------
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        u32x4 pw;
#pragma unroll
        for (int s = 0; s < 4; ++s) pw[s] = T::pack2(sacc[kb][8 * g + 2 * s], sacc[kb][8 * g + 2 * s + 1]);
        const vec8 pb = as_vec8<vec8>(pw);
        const int kc = 32 * kb + 16 * g + 4 * hf;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint16_t* vr = &vt[(32 * db + lr) * VT + kc];
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vr);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vr + 8);
          const u32x4 aw = {lo[0], lo[1], hi[0], hi[1]};
          oacc[db] = T::mfma32(as_vec8<vec8>(aw), pb, oacc[db]);
        }
      }
    }
  }

  // ---- epilogue -------------------------------------------------------------
  const float l = l_run + wave_shfl_xor(l_run, 32);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (qvalid) {
    uint16_t* orow = p.o + (int64_t)b * p.o_s[0] + (int64_t)h * p.o_s[1] + (int64_t)qi * p.o_s[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * hf;
        if (d0 < D) {
          u32x2 w;
          w[0] = T::pack2(oacc[db][4 * g] * inv, oacc[db][4 * g + 1] * inv);
          w[1] = T::pack2(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv);
          *reinterpret_cast<u32x2*>(orow + d0) = w;
        }
      }
    if (hf == 0)
      p.lse[((int64_t)b * p.Hq + h) * Nq + qi] =
          m_run == -INFINITY ? -INFINITY : (m_run + __builtin_amdgcn_logf(l)) * kLn2;
  }
}

template <typename T, int EP, int DV>
hipError_t launch_t(const FlashFwdParams& p, hipStream_t s) {
  const int blocks = p.nqb * p.B * p.Hq;
  return launch_named("flash_fwd", flash_fwd_kernel<T, EP, DV>, dim3(blocks), dim3(kFwdThreads), s, p);
}

template <typename T>
hipError_t dispatch(const FlashFwdParams& p, hipStream_t s) {
  const int DV = (p.D + 31) / 32 * 32;
  const int EP = (p.D + p.R + 31) / 32 * 32;
#define POPE_FWD_CASE(ep, dv) \
  if (EP == ep && DV == dv) return launch_t<T, ep, dv>(p, s);
  POPE_FWD_CASE(32, 32) POPE_FWD_CASE(64, 32)
  POPE_FWD_CASE(64, 64) POPE_FWD_CASE(96, 64) POPE_FWD_CASE(128, 64)
  POPE_FWD_CASE(96, 96) POPE_FWD_CASE(128, 96) POPE_FWD_CASE(160, 96) POPE_FWD_CASE(192, 96)
  POPE_FWD_CASE(128, 128) POPE_FWD_CASE(160, 128) POPE_FWD_CASE(192, 128) POPE_FWD_CASE(224, 128)
  POPE_FWD_CASE(256, 128)
#undef POPE_FWD_CASE
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_flash_fwd(const FlashFwdParams& p, int dtype, hipStream_t s) {
  return dtype == 2 ? dispatch<BF16>(p, s) : dispatch<F16>(p, s);
}

}  // namespace pope
