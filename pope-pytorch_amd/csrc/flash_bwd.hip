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
// Q_hat, K_hat, the cos/sin tables and the key visibility words come from the shared
// preparation (flash_prep.hip).  Q_hat is pre-scaled by s = softmax_scale * log2(e), so the
// recomputed score Q_hat K_hat^T is already in log2 units (P = exp2(score - lse * log2 e)) and
// the dK_hat accumulator dS^T Q_hat carries a factor s that the epilogue turns into
// softmax_scale by multiplying with ln 2.
//
// Launches (all on the caller's stream, no atomics except dfreqs / dbias):
//   delta      : -lse * log2 e and -rowsum(O * dO) per query row
//   bwd_main   : one launch holding two kinds of jobs, one per workgroup
//     dK/dV job: 32 keys per wave (256 keys in 8 waves when D + R and D are small,
//                128 in 4 waves otherwise) of one (batch, kv head); loops over the
//                query heads of its group and the query steps (128 rows; 64 for
//                the widest rows) that can see its keys (steps before the causal diagonal are
//                skipped); the epilogue applies the key-side chain rule and sums
//                dbias.
//     dQ job   : 32 queries per wave, the same job sizes; loops over the key
//                steps up to the causal diagonal; the epilogue applies the
//                query-side chain rule.  dQ needs no atomics, so dq is
//                deterministic (the reference accumulates it with atomics in the
//                input dtype, triton_pope_flash_attn.py:215).
//   Causal dK/dV job r and dQ job (blocks - 1 - r) cost the same; the launch
//   orders the pairs heaviest first, so the triangle's work balances over the
//   CUs.  Streamed tiles go straight from global memory into a ring of LDS slots
//   (global_load_lds_dwordx4): three slots, two steps ahead of the step computed, or,
//   for wide rows whose 128-row slots only fit twice, two slots one step ahead.
//   The row terms enter the MFMAs as initial accumulators: the score product
//   starts from -lse (so it returns s - lse and P = exp2 of it) and dO V^T from
//   -delta (so it returns dP - delta).
//
// MFMA layouts (v_mfma_f32_32x32x16, result lane = column, registers = rows
// 8 (r / 4) + 4 half + r % 4): a result read back as an operand has, per 16-wide
// k group, the rows [4 half, 4 half + 4) and [8 + 4 half, 12 + 4 half).  The
// other operand of such a product is read from a row-major LDS tile with
// ds_read_b64_tr_b16 in the same row order (lds_operand_tr), so no transposed
// copy of any tile is ever stored.
#include <type_traits>

#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

typedef const __attribute__((address_space(4))) uint64_t cu64;
typedef const __attribute__((address_space(4))) int ci32;

// Calls f(std::integral_constant<int, n>) for the runtime n in [0, N]: register arrays indexed
// by n stay statically indexed.
template <int N, typename F>
__device__ __forceinline__ void with_const(int n, F&& f) {
  if constexpr (N >= 0) {
    if (n == N) {
      f(std::integral_constant<int, N>{});
      return;
    }
    with_const<N - 1>(n, f);
  }
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
// delta: 8 lanes per (batch * query head, padded query row), one 8-element chunk of O and dO
// each (_bwd_preprocess, triton_pope_flash_attn.py:119-130).  Writes -lse * log2 e and
// -rowsum(O * dO), the initial accumulators of the main kernel's score and dO V^T products;
// rows past Nq and rows with every key masked get -inf, so their P = exp2(s - inf) is 0.
// With `zero_grads` the kernel also clears dfreqs / dbias, which the main kernel accumulates
// into.
template <typename T>
__global__ __launch_bounds__(256) void bwd_delta_kernel(FlashBwdParams p) {
  const int D = p.D, NqP = p.NqP;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p.zero_grads) {
    if (p.dbias && gid < (int64_t)p.Hb * p.R) p.dbias[(gid / p.R) * p.bias_sh + gid % p.R] = 0.f;
    const int64_t ndf = (int64_t)p.Bt * p.Ht * p.Nk * p.R;
    // dense (bt, ht, n, d) layout (the usual one): a flat range, no index decomposition
    const bool dense = p.df_s[2] == p.R && (p.Ht == 1 || p.df_s[1] == (int64_t)p.Nk * p.R) &&
                       (p.Bt == 1 || p.df_s[0] == (int64_t)p.Ht * p.Nk * p.R);
    if (p.dfreqs && dense)
      for (int64_t x = gid; x < ndf; x += (int64_t)gridDim.x * 256) p.dfreqs[x] = 0.f;
    else if (p.dfreqs)
      for (int64_t x = gid; x < ndf; x += (int64_t)gridDim.x * 256) {
        const int d = (int)(x % p.R);
        int64_t rest = x / p.R;
        const int n = (int)(rest % p.Nk);
        rest /= p.Nk;
        const int ht = (int)(rest % p.Ht), bt = (int)(rest / p.Ht);
        p.dfreqs[(int64_t)bt * p.df_s[0] + (int64_t)ht * p.df_s[1] + (int64_t)n * p.df_s[2] + d] = 0.f;
      }
  }
  const int64_t idx = gid >> 3;
  const int part = (int)(gid & 7);
  if (idx >= (int64_t)p.B * p.Hq * NqP) return;   // whole groups of 8 lanes leave together
  const int i = (int)(idx % NqP);
  const int bh = (int)(idx / NqP);
  const int b = bh / p.Hq, h = bh % p.Hq;
  // padding rows (i >= Nq) read the last row and discard it: the loads, the LSE's included, are
  // unconditional and issued together
  const int ic = min(i, p.Nq - 1);
  const float l = p.lse[(int64_t)bh * p.Nq + ic];
  const uint16_t* orow = p.o + (int64_t)b * p.o_s[0] + (int64_t)h * p.o_s[1] + (int64_t)ic * p.o_s[2];
  const uint16_t* drow = p.dout + (int64_t)b * p.do_s[0] + (int64_t)h * p.do_s[1] + (int64_t)ic * p.do_s[2];
  float dl = 0.f;
  for (int d0 = 8 * part; d0 < D; d0 += 64) {
    float xo[8], xd[8];
    unpack8<T>(ld16(orow + d0), xo);
    unpack8<T>(ld16(drow + d0), xd);
#pragma unroll
    for (int s = 0; s < 8; ++s) dl = fmaf(xo[s], xd[s], dl);
  }
  dl += __shfl_xor(dl, 1, 64);
  dl += __shfl_xor(dl, 2, 64);
  dl += __shfl_xor(dl, 4, 64);
  if (part == 0) {
    const bool live = i < p.Nq;
    p.nl[idx] = live && l != -INFINITY ? -l * kLog2e : -INFINITY;
    p.nd[idx] = live ? -dl : 0.f;
  }
}

// ---------------------------------------------------------------------------
template <int EP, int DV>
struct BwdCfg {
  // Small rows: 8 waves (256 keys per dK/dV job, 256 queries per dQ job) and 128-row steps, one
  // workgroup per CU (two waves per SIMD).  Wide rows need up to 512 registers per lane: 4 waves,
  // one per SIMD; 128-row steps in a two-slot ring where two such slots fit (C4's E = 192, D = 96:
  // 326 against 331 us with 64-row steps in three slots), else 64-row steps in three.
  static constexpr bool kBig = EP + DV > 160;
  static constexpr int NW = kBig ? 4 : 8;                    // waves per workgroup
  static constexpr int THREADS = 64 * NW;
  static constexpr int JOB = 32 * NW;                        // keys (dK/dV) or queries (dQ) per job
  // wide rows: 128-row steps in a two-slot ring when two such slots fit the LDS, else 64-row steps in three
  static constexpr bool kWide128 = kBig && 2 * ((128 * EP + 128 * DV) * 2 + 64 * 16) <= 150 * 1024;
  static constexpr int BM = (kBig && !kWide128) ? 64 : 128;  // query rows per dK/dV step, keys per dQ step
  static constexpr int SLOTS = kWide128 ? 2 : 3;
  static constexpr int KS = EP / 16, DS = DV / 16, EB = EP / 32, DB = DV / 32;
  static constexpr int EPU = EP / 8, DVU = DV / 8;
  static constexpr int XT = BM * EP, YT = BM * DV;            // elements of the two tiles of a slot
  static constexpr int XU = XT / 8, YU = YT / 8;              // their 16-byte units
  static constexpr int LU = BM / 2;                           // -lse and -delta rows (dK/dV slot)
  static constexpr int KV_UNITS = XU + YU + LU, Q_UNITS = XU + YU;
  static constexpr int SLOT = KV_UNITS * 16;
  // loads per thread per step, and the count every wave issues (the last load can be partial)
  static constexpr int KV_LPT = (KV_UNITS + THREADS - 1) / THREADS;
  static constexpr int Q_LPT = (Q_UNITS + THREADS - 1) / THREADS;
  static constexpr int KV_LMIN = (KV_UNITS - (THREADS - 64) + THREADS - 1) / THREADS;   // loads of the last wave
  static constexpr int Q_LMIN = (Q_UNITS - (THREADS - 64) + THREADS - 1) / THREADS;
  static constexpr int EPI = 32 * (EP + 1) * 4;
  static constexpr int LDS = SLOTS * SLOT > EPI ? SLOTS * SLOT : EPI;
  static_assert(XU % 64 == 0 && YU % 64 == 0, "tile regions must split at wave boundaries");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

// dK / dV job.  Lane lr of wave w owns key j0 + 32 w + lr.
//   S  = Q_hat K_hat^T - lse : A = Q_hat tile rows (LDS), B = the lane's K_hat row (regs)
//   dP = dO V^T - delta      : A = dO tile rows (LDS),    B = the lane's V row (regs)
// Both results have lane = key, registers = queries, so P and dS are A operands
// (lane = key row, k = queries) of
//   dV     += P^T dO      B = dO tile read transposed
//   dK_hat += dS^T Q_hat  B = Q_hat tile read transposed
template <typename T, int EP, int DV>
__device__ __forceinline__ void dkdv_job(const FlashBwdParams& p, char* smem, float* dbias_s, int kb, int bhk) {
  typedef BwdCfg<EP, DV> C;
  constexpr int BM = C::BM, KS = C::KS, DS = C::DS, EB = C::EB, DB = C::DB, QB = BM / 32;
  constexpr int kThreads = C::THREADS;
  constexpr int EPU = C::EPU, DVU = C::DVU, XU = C::XU, YU = C::YU, UNITS = C::KV_UNITS;
  typedef typename T::vec8 vec8;

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int b = bhk / p.Hk, hk = bhk % p.Hk;
  const int D = p.D, R = p.R, Nq = p.Nq, Nk = p.Nk, NqP = p.NqP;
  const int j0 = kb * C::JOB;
  const int kw0 = j0 + 32 * wave;   // first key of this wave
  const int kj = kw0 + lr;

  cu64* mw = (cu64*)p.mwords + (int64_t)b * p.NW;
  const uint64_t kword = mw[kj >> 6];   // kj < NkP: a word exists
  const bool kvis = (kword >> (kj & 63)) & 1ull;
  for (int e = tid; e < EP; e += kThreads) dbias_s[e] = 0.f;

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
  settle_vector_loads();

  f32x16 dva[DB], dka[EB];
#pragma unroll
  for (int x = 0; x < DB; ++x)
#pragma unroll
    for (int r = 0; r < 16; ++r) dva[x][r] = 0.f;
#pragma unroll
  for (int x = 0; x < EB; ++x)
#pragma unroll
    for (int r = 0; r < 16; ++r) dka[x][r] = 0.f;

  const bool wave_vis = __all(kvis);
  const bool wave_any = __any(kvis);
  const int any_key = __syncthreads_or(kvis ? 1 : 0);
  const int nqt = NqP / BM;
  const int qt0 = p.causal ? j0 / BM : 0;
  const int groups = p.Hq / p.Hk;
  const int per_head = nqt - qt0;
  const int nsteps = any_key ? groups * per_head : 0;

  // ---- direct-load plan: unit c = m * 256 + tid of a slot (Q_hat tile | dO tile | -lse | -delta)
  const uint16_t* qh_job = p.qh + (int64_t)(b * p.Hq + hk) * NqP * EP;
  const int64_t qh_hstride = (int64_t)p.Hk * NqP * EP;
  const uint16_t* do_job = p.dout + (int64_t)b * p.do_s[0] + (int64_t)hk * p.do_s[1];
  const int64_t do_hstride = (int64_t)p.Hk * p.do_s[1];
  const int do_rs = (int)p.do_s[2];
  const float* nl_job = p.nl + (int64_t)(b * p.Hq + hk) * NqP;
  const int64_t nl_hstride = (int64_t)p.Hk * NqP;
  // one offset per load: Q_hat element offset in the tile; dO element offset of (row, column)
  // relative to the tile's first row (rows past Nq clamp to the last chunk of the last row:
  // those rows only meet P = 0); -lse / -delta offset from the tile's first -lse row (the -delta array
  // follows the -lse array in the workspace)
  const int64_t nd_off = p.nd - p.nl;
  int ld_o[C::KV_LPT];
#pragma unroll
  for (int m = 0; m < C::KV_LPT; ++m) {
    const int c = m * kThreads + tid;
    if (c < XU) {
      const int r = c / EPU;
      ld_o[m] = r * EP + 8 * ((c % EPU) ^ tile_swz(EPU, r));
    } else if (c < XU + YU) {
      const int r = (c - XU) / DVU;
      ld_o[m] = r * do_rs + min(8 * (((c - XU) % DVU) ^ tile_swz(DVU, r)), D - 8);
    } else {
      const int cl = c - XU - YU;   // 4 rows per unit: -lse rows, then -delta rows
      ld_o[m] = 4 * (cl % (BM / 4)) + (cl < BM / 4 ? 0 : (int)nd_off);
    }
  }
  const int do_last = (Nq - 1) * do_rs + D - 8;   // start of the last chunk of the last row
  auto issue = [&](int st) {
    const int g = st / per_head, i0 = (qt0 + st % per_head) * BM;
    char* slot = smem + (st % C::SLOTS) * C::SLOT;
    const uint16_t* qg = qh_job + g * qh_hstride + (int64_t)i0 * EP;
    const uint16_t* dg = do_job + g * do_hstride;
    const float* lg = nl_job + g * nl_hstride + i0;
    const int drow0 = i0 * do_rs;
#pragma unroll
    for (int m = 0; m < C::KV_LPT; ++m) {
      const int c0 = m * kThreads + wave * 64;
      const uint32_t dst = lds_addr(slot + c0 * 16);
      if ((m + 1) * kThreads <= XU) {
        load_lds16(qg + ld_o[m], dst);
      } else if (m * kThreads >= XU && (m + 1) * kThreads <= XU + YU) {
        load_lds16(dg + min(drow0 + ld_o[m], do_last), dst);
      } else {   // boundary loads: per-wave region, partial waves past the slot
        if (c0 < XU) {
          load_lds16(qg + ld_o[m], dst);
        } else if (c0 < XU + YU) {
          load_lds16(dg + min(drow0 + ld_o[m], do_last), dst);
        } else if (c0 < UNITS) {
          if (m * kThreads + tid < UNITS) load_lds16(lg + ld_o[m], dst);
        }
      }
    }
  };

  // ---- LDS operand offsets (elements) ------------------------------------------------
  const TileOffsets<EPU> qo(lane);
  const TileOffsets<DVU> doo(lane);

  constexpr int PD = C::SLOTS - 1;   // steps in flight ahead of the one computed
  if (nsteps > 0) issue(0);
  if (PD > 1 && nsteps > 1) issue(1);
  for (int st = 0; st < nsteps; ++st) {
    if constexpr (PD > 1) {
      if (st + 1 < nsteps) wait_vmcnt<C::KV_LMIN>();   // this thread's loads of step st landed
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();                                // ... everyone's; step st - 1's slot is free
    if (st + PD < nsteps) issue(st + PD);
    const int i0 = (qt0 + st % per_head) * BM;
    // byte addresses in the step's slot: Q_hat tile | dO tile | -lse rows | -delta rows
    const uint32_t sb = lds_addr(smem + (st % C::SLOTS) * C::SLOT);
    const TileAddr<EPU> qa(qo, sb);
    const TileAddr<DVU> da(doo, sb + 2 * C::XT);
    const uint32_t nla = opaque_u32(sb + 2 * (C::XT + C::YT) + 16 * hf);
#pragma unroll
    for (int qs = 0; qs < QB; ++qs) {
      // every query of the sub-tile before every key of the wave (causal), or no visible key
      if ((p.causal && i0 + 32 * qs + 31 < kw0) || !wave_any) continue;
      f32x16 s, dp;
#pragma unroll
      for (int q = 0; q < 4; ++q) {   // rows 32 qs + 8 q + 4 hf + (0..3)
        const f32x4 a = lds_read_f4_at(nla + 4 * (32 * qs + 8 * q));
        const f32x4 d = lds_read_f4_at(nla + 4 * (BM + 32 * qs + 8 * q));
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          s[4 * q + x] = a[x];
          dp[4 * q + x] = d[x];
        }
      }
      // every operand read of the two products issued before the first product, so one LDS
      // latency is exposed per sub-tile instead of one per product
      u32x4 fq[KS], fd[DS];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) fq[kk] = lds_read16_at(qa.row_at(kk) + 2 * 32 * qs * EP);
#pragma unroll
      for (int kk = 0; kk < DS; ++kk) fd[kk] = lds_read16_at(da.row_at(kk) + 2 * 32 * qs * DV);
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) s = T::mfma32(as_vec8<vec8>(fq[kk]), kreg[kk], s);
#pragma unroll
      for (int kk = 0; kk < DS; ++kk) dp = T::mfma32(as_vec8<vec8>(fd[kk]), vreg[kk], dp);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8 + KS + DS, 0);   // with the 8 row-term reads
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, KS + DS, 0);
      // Partial sub-tile (some key of the wave masked, or on the causal diagonal): masked
      // scores become -inf so that P = 0.
      if (!wave_vis || (p.causal && i0 + 32 * qs < kw0 + 31)) {
        POPE_COLD_PATH();
        const int lim = i0 + 32 * qs + 4 * hf - kj;   // causal: row offset >= -lim
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qr = 8 * (r >> 2) + (r & 3);
          s[r] = (kvis && (!p.causal || qr + lim >= 0)) ? s[r] : -INFINITY;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = __builtin_amdgcn_exp2f(s[r]);
        s[r] = pv;
        dp[r] = pv * dp[r];
      }
      // The two waves of a SIMD run this loop in step between the barriers, so their product
      // bursts and their exponentials would coincide.  Raised priority for the dV / dK burst lets
      // the wave that reaches it first keep the matrix pipe; the other wave's exponentials and
      // packs then run beside it, and the two drift half a sub-tile apart (8-wave workgroups only:
      // with one wave per SIMD there is nothing to arbitrate).
      if constexpr (C::NW == 8) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const vec8 ap = as_vec8<vec8>(pack8<T>(s, g2));
        const vec8 ads = as_vec8<vec8>(pack8<T>(dp, g2));
        const int r0 = 32 * qs + 16 * g2;
#pragma unroll
        for (int db = 0; db < DB; ++db)
          dva[db] = T::mfma32(ap, as_vec8<vec8>(lds_tr8_at(da.lo_at(db) + 2 * r0 * DV, da.hi_at(db) + 2 * r0 * DV)),
                              dva[db]);
#pragma unroll
        for (int eb = 0; eb < EB; ++eb)
          dka[eb] = T::mfma32(ads, as_vec8<vec8>(lds_tr8_at(qa.lo_at(eb) + 2 * r0 * EP, qa.hi_at(eb) + 2 * r0 * EP)),
                              dka[eb]);
      }
      if constexpr (C::NW == 8) __builtin_amdgcn_s_setprio(0);
    }
  }
  __syncthreads();   // every wave is done with the slots

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

  // ---- dK: key-side chain rule ---------------------------------------------------
  // dka lane lr of block eb holds column e = 32 eb + lr of dK_hat for the wave's 16 keys
  // 8 (r >> 2) + 4 hf + (r & 3).  With R a multiple of 32 the cos column of dim d < R (e = d)
  // and its sin column (e = R + d) sit in the same lane, blocks eb and eb + R / 32, and a
  // pass-through dim d >= R (e = R + d) in block (R + d) / 32: the chain rule runs on the
  // registers, with every load of the lane issued before the arithmetic.
  const uint16_t* kb_ptr = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1];
  uint16_t* dkb = p.dk + (int64_t)b * p.dk_s[0] + (int64_t)hk * p.dk_s[1];
  const float2* tb = R ? p.table + (int64_t)b * p.t_sb + (int64_t)hk * p.t_sh : nullptr;
  float* dfb = p.dfreqs ? p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)hk * p.df_s[1] : nullptr;
  // deterministic mode: each key's dpsi is written once, summed later in a fixed order
  float* kpb = p.kpart ? p.kpart + (int64_t)(b * p.Hk + hk) * Nk * R : nullptr;
  if (R % 32 == 0) {
    auto key_of = [&](int r) { return kw0 + 8 * (r >> 2) + 4 * hf + (r & 3); };
    with_const<EP / 64>(R / 32, [&](auto rbc) {   // rotated blocks: R / 32 <= EP / 64
    constexpr int RB = decltype(rbc)::value;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int d = 32 * rb + lr;
      float x[16];
      float2 cs[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = min(key_of(r), Nk - 1);
        x[r] = T::to_float(kb_ptr[(int64_t)key * p.k_s[2] + d]);
        cs[r] = tb[(int64_t)key * R + d];
      }
      float dsum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float uc = dka[rb][r] * kLn2, us = dka[rb + RB][r] * kLn2;
        const float g = sigmoid_f(x[r]) * (cs[r].x * uc + cs[r].y * us);
        const float dpsi = softplus_f(x[r]) * (cs[r].x * us - cs[r].y * uc);
        const int key = key_of(r);
        if (key < Nk) {
          dkb[(int64_t)key * p.dk_s[2] + d] = T::bits(g);
          if (kpb) kpb[(int64_t)key * R + d] = dpsi;
          else if (dfb) atomicAdd(dfb + (int64_t)key * p.df_s[2] + d, dpsi);
          dsum += dpsi;
        }
      }
      if (p.dbias && !kpb) {
        dsum += wave_shfl_xor(dsum, 32);
        if (hf == 0) atomicAdd(&dbias_s[d], dsum);
      }
    }
#pragma unroll
    for (int eb = 2 * RB; eb < EB; ++eb) {   // pass-through dims
      const int d = 32 * eb + lr - R;
      if (d >= D) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = key_of(r);
        if (key < Nk) dkb[(int64_t)key * p.dk_s[2] + d] = T::bits(dka[eb][r] * kLn2);
      }
    }
    });
  } else {
    // general rotate dim: one wave's 32 keys at a time through LDS
    constexpr int BS = EP + 1;
    float* ebuf = reinterpret_cast<float*>(smem);
    for (int w = 0; w < C::NW; ++w) {
      __syncthreads();
      if (wave == w) {
  #pragma unroll
        for (int eb = 0; eb < EB; ++eb)
  #pragma unroll
          for (int r = 0; r < 16; ++r) ebuf[(8 * (r >> 2) + 4 * hf + (r & 3)) * BS + 32 * eb + lr] = dka[eb][r];
      }
      __syncthreads();
      for (int it = tid; it < 32 * D; it += kThreads) {
        const int kr = it / D, d = it - kr * D;
        const int key = j0 + 32 * w + kr;
        if (key >= Nk) continue;
        const float* row = ebuf + kr * BS;
        float g;
        if (d < R) {
          const float x = T::to_float(kb_ptr[(int64_t)key * p.k_s[2] + d]);
          const float2 cs = tb[(int64_t)key * R + d];
          const float uc = row[d] * kLn2, us = row[R + d] * kLn2;
          g = sigmoid_f(x) * (cs.x * uc + cs.y * us);
          const float dpsi = softplus_f(x) * (cs.x * us - cs.y * uc);
          if (kpb) {
            kpb[(int64_t)key * R + d] = dpsi;
          } else {
            if (dfb) atomicAdd(dfb + (int64_t)key * p.df_s[2] + d, dpsi);
            if (p.dbias) atomicAdd(&dbias_s[d], dpsi);
          }
        } else {
          g = row[R + d] * kLn2;
        }
        dkb[(int64_t)key * p.dk_s[2] + d] = T::bits(g);
      }
    }
  }
  if (p.dbias && !kpb) {
    __syncthreads();
    for (int d = tid; d < R; d += C::THREADS) atomicAdd(p.dbias + (int64_t)hk * p.bias_sh + d, dbias_s[d]);
  }
}

// dQ job.  Lane lr of wave w owns query i0 + 32 w + lr.
//   S^T  = K_hat Q_hat^T - lse : A = K_hat tile rows (LDS), B = the lane's Q_hat row (regs)
//   dP^T = V dO^T - delta      : A = V tile rows (LDS),     B = the lane's dO row (regs)
// Results: lane = query, registers = keys; dS^T is the B operand of
//   dQ_hat^T += K_hat^T dS^T   A = K_hat tile read transposed.
template <typename T, int EP, int DV>
__device__ __forceinline__ void dq_job(const FlashBwdParams& p, char* smem, int qb, int bh) {
  typedef BwdCfg<EP, DV> C;
  constexpr int BN = C::BM, KS = C::KS, DS = C::DS, EB = C::EB, NB = BN / 32;
  constexpr int kThreads = C::THREADS;
  constexpr int EPU = C::EPU, DVU = C::DVU, XU = C::XU, UNITS = C::Q_UNITS;
  typedef typename T::vec8 vec8;

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int bhk = b * p.Hk + hk;
  const int D = p.D, R = p.R, Nq = p.Nq, Nk = p.Nk, NkP = p.NkP;
  const int q_off = Nk - Nq;
  const int qw0 = qb * C::JOB + 32 * wave;
  const int qi = qw0 + lr;

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
      doreg[kk] = as_vec8<vec8>((qi < Nq && d0 < D) ? ld16(dr + d0) : zero4());
    }
  }
  // initial accumulators: -lse and -delta of the lane's query in every register
  f32x16 nlc, ndc;
  {
    const float a = p.nl[(int64_t)bh * p.NqP + qi], d = p.nd[(int64_t)bh * p.NqP + qi];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      nlc[r] = a;
      ndc[r] = d;
    }
  }
  settle_vector_loads();

  f32x16 dqa[EB];
#pragma unroll
  for (int x = 0; x < EB; ++x)
#pragma unroll
    for (int r = 0; r < 16; ++r) dqa[x][r] = 0.f;

  cu64* mw = (cu64*)p.mwords + (int64_t)b * p.NW;
  int nkeys = min(((ci32*)p.kend)[b], Nk);
  if (p.causal) nkeys = min(nkeys, min(qb * C::JOB + C::JOB, Nq));
  const int nt = (nkeys + BN - 1) / BN;

  // ---- direct-load plan: unit c = m * 256 + tid of a slot (K_hat tile | V tile) --------
  const uint16_t* kh_g = p.kh + (int64_t)bhk * NkP * EP;
  const uint16_t* v_g = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  const int vs2 = (int)p.v_s[2];
  // one offset per load: K_hat element offset in the tile; V element offset of (row, column)
  // relative to the tile's first row (rows past Nk clamp to the last chunk of the last row: P = 0 there)
  int ld_o[C::Q_LPT];
#pragma unroll
  for (int m = 0; m < C::Q_LPT; ++m) {
    const int c = m * kThreads + tid;
    if (c < XU) {
      const int r = c / EPU;
      ld_o[m] = r * EP + 8 * ((c % EPU) ^ tile_swz(EPU, r));
    } else {
      const int r = (c - XU) / DVU;
      ld_o[m] = r * vs2 + min(8 * (((c - XU) % DVU) ^ tile_swz(DVU, r)), D - 8);
    }
  }
  const int v_last = (Nk - 1) * vs2 + D - 8;   // start of the last chunk of the last row
  auto issue = [&](int kt) {
    const int j0 = kt * BN;
    char* slot = smem + (kt % C::SLOTS) * C::SLOT;
    const uint16_t* kg = kh_g + j0 * EP;   // K_hat rows are padded to NkP
    const int vrow0 = j0 * vs2;
#pragma unroll
    for (int m = 0; m < C::Q_LPT; ++m) {
      const int c0 = m * kThreads + wave * 64;
      const uint32_t dst = lds_addr(slot + c0 * 16);
      const uint16_t* vsrc = v_g + min(vrow0 + ld_o[m], v_last);
      if ((m + 1) * kThreads <= XU) {
        load_lds16(kg + ld_o[m], dst);
      } else if (m * kThreads >= XU) {
        if (UNITS % kThreads == 0 || c0 < UNITS) load_lds16(vsrc, dst);
      } else {
        load_lds16(c0 < XU ? (const void*)(kg + ld_o[m]) : (const void*)vsrc, dst);
      }
    }
  };

  const TileOffsets<EPU> ko(lane);
  const TileOffsets<DVU> vo(lane);

  constexpr int PD = C::SLOTS - 1;
  if (nt > 0) issue(0);
  if (PD > 1 && nt > 1) issue(1);
  for (int kt = 0; kt < nt; ++kt) {
    if constexpr (PD > 1) {
      if (kt + 1 < nt) wait_vmcnt<C::Q_LMIN>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();
    if (kt + PD < nt) issue(kt + PD);
    const int j0 = kt * BN;
    const uint32_t sb = lds_addr(smem + (kt % C::SLOTS) * C::SLOT);   // K_hat tile | V tile
    const TileAddr<EPU> ka(ko, sb);
    const TileAddr<DVU> va(vo, sb + 2 * C::XT);
#pragma unroll
    for (int ks = 0; ks < NB; ++ks) {
      const int k0 = j0 + 32 * ks;   // first key of the sub-tile
      const uint32_t mb = (uint32_t)(mw[k0 >> 6] >> (k0 & 32));
      // nothing visible to this wave: every key masked, or (causal) after the wave's last query
      if (mb == 0 || (p.causal && k0 > qw0 + 31)) continue;
      // every key visible and (causal) at or before the wave's first query
      const bool full = mb == 0xffffffffu && !(p.causal && k0 + 31 > qw0);
      f32x16 s = nlc, dp = ndc;
      u32x4 fk[KS], fv[DS];   // operand reads first (one exposed LDS latency per sub-tile)
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) fk[kk] = lds_read16_at(ka.row_at(kk) + 2 * 32 * ks * EP);
#pragma unroll
      for (int kk = 0; kk < DS; ++kk) fv[kk] = lds_read16_at(va.row_at(kk) + 2 * 32 * ks * DV);
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) s = T::mfma32(as_vec8<vec8>(fk[kk]), qreg[kk], s);
#pragma unroll
      for (int kk = 0; kk < DS; ++kk) dp = T::mfma32(as_vec8<vec8>(fv[kk]), doreg[kk], dp);
      // the transposed K_hat operands of dQ, read while the products and the exponentials run
      u32x4 ft[2][EB];
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
        for (int eb = 0; eb < EB; ++eb) {
          const uint32_t r0 = 2 * (32 * ks + 16 * g2) * EP;
          ft[g2][eb] = lds_tr8_at(ka.lo_at(eb) + r0, ka.hi_at(eb) + r0);
        }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, KS + DS, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, KS + DS, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4 * EB, 0);
      if (!full) {   // masked scores -> -inf: P = 0
        POPE_COLD_PATH();
        const uint32_t w = mb >> (4 * hf);
        const int lim = p.causal ? qi - k0 - 4 * hf : 64;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kr = 8 * (r >> 2) + (r & 3);
          s[r] = (((w >> kr) & 1u) && kr <= lim) ? s[r] : -INFINITY;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] = __builtin_amdgcn_exp2f(s[r]) * dp[r];
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const vec8 bds = as_vec8<vec8>(pack8<T>(dp, g2));
#pragma unroll
        for (int eb = 0; eb < EB; ++eb) dqa[eb] = T::mfma32(as_vec8<vec8>(ft[g2][eb]), bds, dqa[eb]);
      }
    }
  }
  __syncthreads();   // every wave is done with the slots

  // ---- dQ: query-side chain rule --------------------------------------------------
  // dqa lane (query qi, hf) of block eb holds rows e = 32 eb + 8 (r >> 2) + 4 hf + (r & 3) of
  // dQ_hat^T: with R a multiple of 32, dim d < R has its cos row (e = d) and sin row (e = R + d)
  // in blocks eb and eb + R / 32 at the same register, and pass-through dims d >= R (e = R + d)
  // fill the later blocks.  Each register group of 4 covers 4 consecutive dims.
  const uint16_t* qb_ptr = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1];
  uint16_t* dqb = p.dq + (int64_t)b * p.dq_s[0] + (int64_t)h * p.dq_s[1];
  const float2* tq = R ? p.table + (int64_t)b * p.t_sb + (int64_t)h * p.t_sh : nullptr;
  const float2* bq = R ? p.btab + (p.Hb > 1 ? hk : 0) * R : nullptr;
  float* dfb = p.dfreqs ? p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)h * p.df_s[1] : nullptr;
  // deterministic mode: each query's dphi is written once, summed later in a fixed order
  float* qpb = p.qpart && p.dfreqs ? p.qpart + (int64_t)(b * p.Hq + h) * Nq * R : nullptr;
  if (R % 32 == 0) {
    if (qi < Nq) {
      uint16_t* dqrow = dqb + (int64_t)qi * p.dq_s[2];
      with_const<EP / 64>(R / 32, [&](auto rbc) {   // rotated blocks: R / 32 <= EP / 64
      constexpr int RB = decltype(rbc)::value;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float x[16];
        float2 tf[16], tbv[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * rb + 8 * g + 4 * hf;
          const u32x2 raw = *reinterpret_cast<const u32x2*>(qb_ptr + (int64_t)qi * p.q_s[2] + d0);
          x[4 * g] = T::to_float((uint16_t)u16lo(raw[0]));
          x[4 * g + 1] = T::to_float((uint16_t)u16hi(raw[0]));
          x[4 * g + 2] = T::to_float((uint16_t)u16lo(raw[1]));
          x[4 * g + 3] = T::to_float((uint16_t)u16hi(raw[1]));
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            tf[4 * g + c] = tq[(int64_t)(q_off + qi) * R + d0 + c];
            tbv[4 * g + c] = bq[d0 + c];
          }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * rb + 8 * g + 4 * hf;
          float out[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int r = 4 * g + c;
            // cos / sin(F[q_off + i] - bias) from the tables of F and of the bias
            const float cs = fmaf(tf[r].x, tbv[r].x, tf[r].y * tbv[r].y);
            const float sn = fmaf(tf[r].y, tbv[r].x, -tf[r].x * tbv[r].y);
            const float uc = dqa[rb][r] * p.scale, us = dqa[rb + RB][r] * p.scale;
            out[c] = sigmoid_f(x[r]) * (cs * uc + sn * us);
            const float dph = softplus_f(x[r]) * (cs * us - sn * uc);
            if (qpb) qpb[(int64_t)qi * R + d0 + c] = dph;
            else if (dfb) atomicAdd(dfb + (int64_t)(q_off + qi) * p.df_s[2] + d0 + c, dph);
          }
          u32x2 w;
          w[0] = T::pack2(out[0], out[1]);
          w[1] = T::pack2(out[2], out[3]);
          *reinterpret_cast<u32x2*>(dqrow + d0) = w;
        }
      }
#pragma unroll
      for (int eb = 2 * RB; eb < EB; ++eb) {   // pass-through dims
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * eb + 8 * g + 4 * hf - R;
          if (d0 >= D) continue;
          u32x2 w;
          w[0] = T::pack2(dqa[eb][4 * g] * p.scale, dqa[eb][4 * g + 1] * p.scale);
          w[1] = T::pack2(dqa[eb][4 * g + 2] * p.scale, dqa[eb][4 * g + 3] * p.scale);
          *reinterpret_cast<u32x2*>(dqrow + d0) = w;
        }
      }
      });
    }
  } else {
    // general rotate dim: one wave's 32 queries at a time through LDS
    constexpr int BS = EP + 1;
    float* ebuf = reinterpret_cast<float*>(smem);
    for (int w = 0; w < C::NW; ++w) {
      __syncthreads();
      if (wave == w) {
  #pragma unroll
        for (int eb = 0; eb < EB; ++eb)
  #pragma unroll
          for (int r = 0; r < 16; ++r) ebuf[lr * BS + 32 * eb + 8 * (r >> 2) + 4 * hf + (r & 3)] = dqa[eb][r];
      }
      __syncthreads();
      for (int it = tid; it < 32 * D; it += kThreads) {
        const int qr = it / D, d = it - qr * D;
        const int i = qb * C::JOB + 32 * w + qr;
        if (i >= Nq) continue;
        const float* row = ebuf + qr * BS;
        float g;
        if (d < R) {
          const float x = T::to_float(qb_ptr[(int64_t)i * p.q_s[2] + d]);
          // cos / sin(F[q_off + i] - bias) from the tables of F and of the bias
          const float2 tf = tq[(int64_t)(q_off + i) * R + d], tb = bq[d];
          const float cs = fmaf(tf.x, tb.x, tf.y * tb.y), sn = fmaf(tf.y, tb.x, -tf.x * tb.y);
          const float uc = row[d] * p.scale, us = row[R + d] * p.scale;
          g = sigmoid_f(x) * (cs * uc + sn * us);
          const float dph = softplus_f(x) * (cs * us - sn * uc);
          if (qpb) qpb[(int64_t)i * R + d] = dph;
          else if (dfb) atomicAdd(dfb + (int64_t)(q_off + i) * p.df_s[2] + d, dph);
        } else {
          g = row[R + d] * p.scale;
        }
        dqb[(int64_t)i * p.dq_s[2] + d] = T::bits(g);
      }
    }
  }
}

template <typename T, int EP, int DV>
__global__ __launch_bounds__((BwdCfg<EP, DV>::THREADS), 1) void bwd_main_kernel(FlashBwdParams p) {
  __shared__ __attribute__((aligned(16))) char smem[BwdCfg<EP, DV>::LDS];
  __shared__ float dbias_s[EP];
  const int nqb = p.NqP / BwdCfg<EP, DV>::JOB;
  const int id = blockIdx.x;
  int kind, blk, head;   // kind 0 = dK/dV job (head = b * Hk + hk), 1 = dQ job (head = b * Hq + h)
  if (p.interleave) {
    // pairs of equal cost, heaviest first: dK/dV block r with dQ block nqb - 1 - r; the
    // batch * head index is fastest so that one head's jobs share an XCD (workgroup ids are
    // dealt round-robin over the 8 XCDs).  Workgroups are dispatched in id order, and inside an
    // XCD the ids go round-robin to its shader engines: with the kind fixed by one id bit, each
    // engine held jobs of one kind only, the dQ engines' CUs finished their first jobs 30 us
    // earlier and then waited, because the next id in line belonged to a dK/dV engine without a
    // free CU.  The kind therefore flips with the parity of the head index and of the level, so
    // that every run of ids mixes both kinds.
    const int BH = p.B * p.Hq;
    const int r = id / (2 * BH), rem = id % (2 * BH);
    head = rem % BH;
    kind = (rem / BH) ^ (__builtin_popcount(head) & 1) ^ (r & 1);
    blk = kind == 0 ? r : nqb - 1 - r;
  } else if (id < p.n_kv_jobs) {
    const int BHk = p.B * p.Hk;
    kind = 0;
    blk = id / BHk;
    head = id % BHk;
  } else {
    const int BH = p.B * p.Hq, j = id - p.n_kv_jobs;
    kind = 1;
    blk = p.causal ? nqb - 1 - j / BH : j / BH;
    head = j % BH;
  }
  if (kind == 0)
    dkdv_job<T, EP, DV>(p, smem, dbias_s, blk, head);
  else
    dq_job<T, EP, DV>(p, smem, blk, head);
}

template <typename T, int EP, int DV>
hipError_t launch_t(const FlashBwdParams& p0, hipStream_t s) {
  FlashBwdParams p = p0;
  const int64_t nrows = (int64_t)p.B * p.Hq * p.NqP;
  hipError_t e = launch_named("flash_bwd_delta", bwd_delta_kernel<T>, dim3((unsigned)((8 * nrows + 255) / 256)),
                              dim3(256), s, p);
  if (e != hipSuccess) return e;
  typedef BwdCfg<EP, DV> C;
  const int nkb = p.NkP / C::JOB, nqb = p.NqP / C::JOB;
  p.n_kv_jobs = nkb * p.B * p.Hk;
  p.interleave = p.causal && p.Hq == p.Hk && nkb == nqb && p.Nq == p.Nk;
  const int jobs = p.n_kv_jobs + nqb * p.B * p.Hq;
  return launch_named("flash_bwd", bwd_main_kernel<T, EP, DV>, dim3(jobs), dim3(C::THREADS), s, p);
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

hipError_t launch_flash_bwd_delta(const FlashBwdParams& p, int dtype, hipStream_t s) {
  const int64_t nrows = (int64_t)p.B * p.Hq * p.NqP;
  const dim3 grid((unsigned)((8 * nrows + 255) / 256));
  return dtype == 2 ? launch_named("flash_bwd_delta", bwd_delta_kernel<BF16>, grid, dim3(256), s, p)
                    : launch_named("flash_bwd_delta", bwd_delta_kernel<F16>, grid, dim3(256), s, p);
}

}  // namespace pope
