// Flash attention forward with PoPE fused in (bf16 / fp16 MFMA, gfx950).
//
// Reference semantics: triton_pope_flash_attn.py:23-117 (kernel) and :222-271
// (launcher); PyTorch path attention.py:106-145.
//
// Two launches:
//   fwd_prep_k : K_hat = the polar transform of the keys, written once per call
//                as (B, Hk, NkP, EP) 16-bit rows (zero past Nk and past E);
//   flash_fwd  : the attention sweep.
//
// flash_fwd work decomposition
//   one workgroup = 8 waves = 128 query rows of one (batch, query head).  Waves
//   0-3 (group 0) and 4-7 (group 1) own the same 128 rows, 32 per wave, and
//   split the key axis: per iteration the workgroup stages a pair of 64-key
//   tiles in LDS, group g takes tile 2 t + g.  Each group keeps its own online
//   softmax state; group 1 hands (m, l, O) to group 0 through LDS at the end.
//   The next pair of tiles is fetched into registers while the current pair is
//   computed (LDS double-buffered when it fits the 160 KB of a CU).
// Per tile and wave
//   S^T = K_hat Q_hat^T on v_mfma_f32_32x32x16: A = K_hat tile rows (lane =
//   key), B = the wave's Q_hat held in registers (lane = query).  The result
//   has one query per lane and keys in registers, so the softmax row
//   reductions stay in-lane (plus one swap between the two lane halves).
//   O^T += V^T P^T reuses the probabilities straight from the S registers as
//   the B operand (a key permutation inside each 16-key group); the A operand
//   comes from the row-major V tile through LDS transpose reads in the same key
//   order.  Tiles with every key visible to every row of the wave skip the
//   per-element masks, and the accumulator is rescaled only when a row's
//   running max moves.
// Scheduling
//   blockIdx -> (query block, batch*head) with the heaviest causal blocks first
//   and batch*head fastest, so consecutive workgroups land on different XCDs
//   while every workgroup of one (batch, head) lands on the same XCD (the
//   dispatcher deals workgroup ids round-robin over the 8 XCDs): its K_hat / V
//   stay in one L2.  One workgroup per CU; twice as many workgroups as CUs keep
//   the causal triangle balanced.
// Phases
//   The learned bias is moved to the query side: cos(phi - (F_j + b)) =
//   cos((phi - b) - F_j), so Q_hat = a * (cos, sin)(F[q_off+i] - b) is computed
//   with accurate sincos and K_hat = c * (cos, sin)(F_j) uses the per-call table
//   of cos/sin(F).  Differences to the reference's fl(F_j + b) rounding are
//   below bf16 resolution.
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

constexpr int kBM = 128;        // query rows per workgroup
constexpr int kBN = 64;         // keys per tile (one tile per wave group per iteration)
constexpr int kThreads = 512;   // 8 waves
constexpr int kLdsMax = 160 * 1024;

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(uint16_t* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// ---------------------------------------------------------------------------
// prep_khat: one thread per (batch * kv head, padded key row, 8-column chunk).
template <typename T>
__global__ __launch_bounds__(256) void prep_khat_kernel(KhatParams p) {
  const int nch = p.EP / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.B * p.Hk * p.NkP * nch) return;
  const int c = (int)(idx % nch);
  const int64_t row = idx / nch;
  const int j = (int)(row % p.NkP);
  const int bhk = (int)(row / p.NkP);
  const int b = bhk / p.Hk, hk = bhk % p.Hk;
  const int R = p.R, E = p.D + p.R, e0 = 8 * c;
  u32x4 w = {0u, 0u, 0u, 0u};
  if (j < p.Nk && e0 < E) {
    const bool is_cos = e0 < R, is_sin = !is_cos && e0 < 2 * R;
    const int d0 = is_cos ? e0 : e0 - R;
    const u32x4 raw = ld16(p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1] + (int64_t)j * p.k_s[2] + d0);
    if (is_cos || is_sin) {
      float x[8];
      unpack8<T>(raw, x);
      const float2* t = p.table + (int64_t)b * p.t_sb + (int64_t)hk * p.t_sh + (int64_t)j * R + d0;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float2 t0 = t[2 * s], t1 = t[2 * s + 1];
        const float a0 = softplus_f(x[2 * s]), a1 = softplus_f(x[2 * s + 1]);
        w[s] = is_cos ? T::pack2(a0 * t0.x, a1 * t1.x) : T::pack2(a0 * t0.y, a1 * t1.y);
      }
    } else {
      w = raw;
    }
  }
  st16(p.kh + ((int64_t)bhk * p.NkP + j) * p.EP + e0, w);
}

// ---------------------------------------------------------------------------
template <typename T, int EP, int DV>
struct FwdCfg {
  static constexpr int KH = 8 * lds_units_rows(EP / 8);   // K_hat row stride: row reads only
  static constexpr int VS = 8 * lds_units_tr(DV / 8);     // V row stride: transpose reads only
  static constexpr int BUF = (2 * kBN * KH + 2 * kBN * VS) * 2;   // bytes of one staged pair
  static constexpr int NBUF = 2 * BUF + 64 <= kLdsMax ? 2 : 1;
  static constexpr int MERGE = 4 * 64 * (2 + 16 * (DV / 32)) * 4;   // group 1's (m, l, O) hand-off
  static constexpr int LDS = NBUF * BUF > MERGE ? NBUF * BUF : MERGE;
  static constexpr int KCH = 2 * kBN * (EP / 8);               // 16-byte K_hat chunks per pair
  static constexpr int KLD = (KCH + kThreads - 1) / kThreads;  // per thread
  static constexpr int VCH = 2 * kBN * (DV / 8);               // 16-byte V chunks per pair
  static constexpr int VLD = (VCH + kThreads - 1) / kThreads;
};

template <typename T, int EP, int DV>
__global__ __launch_bounds__(kThreads, 1) void flash_fwd_kernel(FlashFwdParams p) {
  typedef FwdCfg<T, EP, DV> C;
  constexpr int KS = EP / 16, NDB = DV / 32, KH = C::KH, VS = C::VS;
  typedef typename T::vec8 vec8;

  __shared__ __attribute__((aligned(16))) char smem[C::LDS];
  __shared__ uint64_t mbits_s[2][2];   // [buffer][tile of the pair]: bit j = key j0 + j visible

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int grp = wave >> 2, wq = wave & 3;
  const int BH = p.B * p.Hq;
  const int bh = blockIdx.x % BH;
  const int qb = p.nqb - 1 - (int)(blockIdx.x / BH);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int D = p.D, R = p.R, E = D + R, Nk = p.Nk, Nq = p.Nq;
  const int q_off = Nk - Nq;
  const int qw0 = qb * kBM + wq * 32;   // first query row of this wave
  const int qi = qw0 + lr;
  const bool qvalid = qi < Nq;
  const bool fast_ok = p.scale_log2 > 0.f;   // max commutes with the scale
  const TrLane vtr = tr_lane<false>(C::VS, lane);

  // ---- Q_hat for this lane's query row, in MFMA B-operand order ----------
  vec8 qreg[KS];
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1] + (int64_t)min(qi, Nq - 1) * p.q_s[2];
    const float* frow = R ? p.freqs + (int64_t)b * p.f_s[0] + (int64_t)h * p.f_s[1] +
                                (int64_t)(q_off + min(qi, Nq - 1)) * p.f_s[2]
                          : nullptr;
    const float* brow = R ? p.bias + (int64_t)hk * p.bias_sh : nullptr;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
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

  int nt = (Nk + kBN - 1) / kBN;
  if (p.causal) {
    const int last_q = min(qb * kBM + kBM, Nq) - 1;
    nt = min(nt, last_q / kBN + 1);
  }
  const int npair = (nt + 1) / 2;
  const uint16_t* khg = p.kh + (int64_t)(b * p.Hk + hk) * p.NkP * EP;
  const uint16_t* vg = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  const uint8_t* mrow = p.has_mask ? p.mask + (int64_t)b * p.mask_sb : nullptr;

  // ---- staging of a pair of tiles: global -> registers -> LDS ----------------
  u32x4 kpf[C::KLD], vpf[C::VLD];
  uint64_t mpf = 0;
  auto fetch = [&](int pr) {
    const int j0 = pr * 2 * kBN;
    // Branch-free: keys past Nk clamp to the last row (masked, P = 0) and dims past D to the
    // last chunk (those O columns are never stored).
#pragma unroll
    for (int m = 0; m < C::KLD; ++m) {
      const int c = tid + m * kThreads;
      if (C::KCH % kThreads == 0 || c < C::KCH) kpf[m] = ld16(khg + (int64_t)(j0 + c / (EP / 8)) * EP + 8 * (c % (EP / 8)));
    }
#pragma unroll
    for (int m = 0; m < C::VLD; ++m) {
      const int c = tid + m * kThreads;
      if (C::VCH % kThreads == 0 || c < C::VCH) {
        const int key = min(j0 + c / (DV / 8), Nk - 1), d8 = min(8 * (c % (DV / 8)), D - 8);
        vpf[m] = ld16(vg + (int64_t)key * p.v_s[2] + d8);
      }
    }
    if (wave < 2) {   // wave w: visibility bits of tile w of the pair
      const int key = j0 + tid;
      mpf = __ballot(key < Nk && (!p.has_mask || mrow[key] != 0));
    }
  };
  auto stage = [&](int buf) {
    uint16_t* kh = reinterpret_cast<uint16_t*>(smem + buf * C::BUF);
    uint16_t* vs = kh + 2 * kBN * KH;
#pragma unroll
    for (int m = 0; m < C::KLD; ++m) {
      const int c = tid + m * kThreads;
      if (C::KCH % kThreads == 0 || c < C::KCH) st16(kh + (c / (EP / 8)) * KH + 8 * (c % (EP / 8)), kpf[m]);
    }
#pragma unroll
    for (int m = 0; m < C::VLD; ++m) {
      const int c = tid + m * kThreads;
      if (C::VCH % kThreads == 0 || c < C::VCH) st16(vs + (c / (DV / 8)) * VS + 8 * (c % (DV / 8)), vpf[m]);
    }
    if (wave < 2 && lane == 0) mbits_s[buf][wave] = mpf;
  };

  if (npair > 0) {
    fetch(0);
    stage(0);
  }
  __syncthreads();

  for (int t = 0; t < npair; ++t) {
    const int buf = C::NBUF == 2 ? (t & 1) : 0;
    if (t + 1 < npair) fetch(t + 1);

    const int tile = 2 * t + grp;
    const int j0 = tile * kBN;
    // keys visible to some row of this wave: not all masked, not all after the wave's last query
    const uint64_t mraw = mbits_s[buf][grp];
    const uint64_t mb = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)mraw) |
                        ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(mraw >> 32)) << 32);
    const bool live = tile < nt && mb != 0 && !(p.causal && j0 > qw0 + 31);
    if (live) {
      const uint16_t* kh = reinterpret_cast<const uint16_t*>(smem + buf * C::BUF) + grp * kBN * KH;
      const uint16_t* vs = reinterpret_cast<const uint16_t*>(smem + buf * C::BUF) + 2 * kBN * KH + grp * kBN * VS;

      // ---- S^T = K_hat Q_hat^T ---------------------------------------------
      f32x16 sacc[2] = {{}, {}};
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const vec8 a = as_vec8<vec8>(ld16(kh + (32 * kb + lr) * KH + 16 * kk + 8 * hf));
          sacc[kb] = T::mfma32(a, qreg[kk], sacc[kb]);
        }
      }
      // ---- masks (partial tiles only) + running max -------------------------
      // full tile: every key visible and (causal) every key <= the wave's first query
      const bool full = fast_ok && mb == ~0ull && !(p.causal && j0 + kBN - 1 > qw0);
      float mt = -INFINITY;
      if (full) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[kb][r]);
        mt *= p.scale_log2;
      } else {
        POPE_COLD_PATH();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kr = 32 * kb + 8 * (r >> 2) + 4 * hf + (r & 3);
            const bool ok = ((mb >> kr) & 1ull) && (!p.causal || j0 + kr <= qi);
            const float sv = ok ? sacc[kb][r] * p.scale_log2 : -INFINITY;
            sacc[kb][r] = sv;
            mt = fmaxf(mt, sv);
          }
      }
      mt = fmaxf(mt, wave_shfl_xor(mt, 32));
      const float m_new = fmaxf(m_run, mt);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      if (__any(m_new != m_run)) {   // rescale only when some row's max moved
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
        m_run = m_new;
      }
      float psum = 0.f;
      if (full) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float pr = __builtin_amdgcn_exp2f(fmaf(sacc[kb][r], p.scale_log2, -m_use));
            sacc[kb][r] = pr;
            psum += pr;
          }
      } else {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float pr = __builtin_amdgcn_exp2f(sacc[kb][r] - m_use);
            sacc[kb][r] = pr;
            psum += pr;
          }
      }
      l_run += psum;

      // ---- O^T += V^T P^T: A = V tile read transposed ----------------------
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          u32x4 pw;
#pragma unroll
          for (int s = 0; s < 4; ++s) pw[s] = T::pack2(sacc[kb][8 * g + 2 * s], sacc[kb][8 * g + 2 * s + 1]);
          const vec8 pb = as_vec8<vec8>(pw);
#pragma unroll
          for (int db = 0; db < NDB; ++db)
            oacc[db] = T::mfma32(as_vec8<vec8>(lds_operand_tr(vs, vtr, VS, 32 * kb + 16 * g, 32 * db)), pb, oacc[db]);
        }
      }
    }

    if (t + 1 < npair) {
      if (C::NBUF == 1) __syncthreads();   // every wave is done with the single buffer
      stage(C::NBUF == 2 ? buf ^ 1 : 0);
    }
    __syncthreads();
  }

  // ---- merge group 1 into group 0, epilogue ------------------------------------
  float* mg = reinterpret_cast<float*>(smem);
  constexpr int MS = 2 + 16 * NDB;   // floats per lane in the hand-off
  if (grp == 1) {
    float* dst = mg + (wq * 64 + lane) * MS;
    dst[0] = m_run;
    dst[1] = l_run;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[2 + 16 * db + r] = oacc[db][r];
  }
  __syncthreads();
  if (grp == 1) return;
  {
    const float* src = mg + (wq * 64 + lane) * MS;
    const float m1 = src[0], l1 = src[1];
    const float m_new = fmaxf(m_run, m1);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float a0 = __builtin_amdgcn_exp2f(m_run - m_use), a1 = __builtin_amdgcn_exp2f(m1 - m_use);
    l_run = l_run * a0 + l1 * a1;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] = oacc[db][r] * a0 + src[2 + 16 * db + r] * a1;
  }
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
  KhatParams kp;
  kp.k = p.k;
  kp.k_s[0] = p.k_s[0]; kp.k_s[1] = p.k_s[1]; kp.k_s[2] = p.k_s[2];
  kp.table = p.table;
  kp.t_sb = p.t_sb;
  kp.t_sh = p.t_sh;
  kp.kh = p.kh;
  kp.B = p.B; kp.Hk = p.Hk; kp.Nk = p.Nk; kp.NkP = p.NkP; kp.D = p.D; kp.R = p.R; kp.EP = EP;
  hipError_t e = launch_prep_khat(kp, T::kCode, s);
  if (e != hipSuccess) return e;
  const int blocks = p.nqb * p.B * p.Hq;
  return launch_named("flash_fwd", flash_fwd_kernel<T, EP, DV>, dim3(blocks), dim3(kThreads), s, p);
}

template <typename T>
hipError_t dispatch(const FlashFwdParams& p, hipStream_t s) {
#define POPE_FWD_CASE(ep, dv) \
  if (p.EP == ep && p.DV == dv) return launch_t<T, ep, dv>(p, s);
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

hipError_t launch_prep_khat(const KhatParams& p, int dtype, hipStream_t s) {
  const int64_t n = (int64_t)p.B * p.Hk * p.NkP * (p.EP / 8);
  const dim3 grid((unsigned)((n + 255) / 256));
  return dtype == 2 ? launch_named("prep_khat", prep_khat_kernel<BF16>, grid, dim3(256), s, p)
                    : launch_named("prep_khat", prep_khat_kernel<F16>, grid, dim3(256), s, p);
}

}  // namespace pope
