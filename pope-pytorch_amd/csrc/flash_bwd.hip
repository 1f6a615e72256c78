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
//   delta      : (lse * log2 e, rowsum(O * dO)) per query row
//   bwd_main   : one launch holding two kinds of jobs, one per workgroup of 4 waves
//     dK/dV job: 128 keys (32 per wave) of one (batch, kv head); loops over the
//                query heads of its group and the query tiles that can see its
//                keys (tiles before the causal diagonal are skipped); the
//                epilogue applies the key-side chain rule and sums dbias.
//     dQ job   : 128 queries (32 per wave); loops over the key tiles up to the
//                causal diagonal; the epilogue applies the query-side chain
//                rule.  dQ needs no atomics, so dq is deterministic (the
//                reference accumulates it with atomics in the input dtype,
//                triton_pope_flash_attn.py:215).
//   Causal dK/dV job r and dQ job (blocks - 1 - r) cost the same; the launch
//   orders the pairs heaviest first, so the triangle's work balances over the
//   CUs.  Streamed tiles are double-buffered in LDS, the next one fetched into
//   registers while the current one is computed.
//
// MFMA layouts (v_mfma_f32_32x32x16, result lane = column, registers = rows
// 8 (r / 4) + 4 half + r % 4): a result read back as an operand has, per 16-wide
// k group, the rows [4 half, 4 half + 4) and [8 + 4 half, 12 + 4 half).  The
// other operand of such a product is read from a row-major LDS tile with
// ds_read_b64_tr_b16 in the same row order (lds_operand_tr), so no transposed
// copy of any tile is ever stored.
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(uint16_t* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

// Registers [8 g, 8 g + 8) of an MFMA result, packed as an 8-element operand.
template <typename T>
__device__ __forceinline__ u32x4 pack8(const f32x16& x, int g) {
  u32x4 w;
#pragma unroll
  for (int s = 0; s < 4; ++s) w[s] = T::pack2(x[8 * g + 2 * s], x[8 * g + 2 * s + 1]);
  return w;
}

// ---------------------------------------------------------------------------
// delta: one thread per (batch * query head, padded query row): (lse * log2 e, rowsum(O * dO))
// (_bwd_preprocess, triton_pope_flash_attn.py:119-130).  Rows past Nq and rows with every key
// masked carry lse = +inf, so their P = exp2(s - lse) is 0 without a test.  With `zero_grads`
// the first threads also clear dfreqs / dbias, which the main kernel accumulates into.
template <typename T>
__global__ __launch_bounds__(256) void bwd_delta_kernel(FlashBwdParams p) {
  const int D = p.D, NqP = p.NqP;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p.zero_grads) {
    if (p.dbias && idx < (int64_t)p.Hb * p.R) p.dbias[(idx / p.R) * p.bias_sh + idx % p.R] = 0.f;
    const int64_t ndf = (int64_t)p.Bt * p.Ht * p.Nk * p.R;
    if (p.dfreqs)
      for (int64_t x = idx; x < ndf; x += (int64_t)gridDim.x * 256) {
        const int d = (int)(x % p.R);
        int64_t rest = x / p.R;
        const int n = (int)(rest % p.Nk);
        rest /= p.Nk;
        const int ht = (int)(rest % p.Ht), bt = (int)(rest / p.Ht);
        p.dfreqs[(int64_t)bt * p.df_s[0] + (int64_t)ht * p.df_s[1] + (int64_t)n * p.df_s[2] + d] = 0.f;
      }
  }
  if (idx >= (int64_t)p.B * p.Hq * NqP) return;
  const int i = (int)(idx % NqP);
  const int bh = (int)(idx / NqP);
  const int b = bh / p.Hq, h = bh % p.Hq;
  float dl = 0.f, l2 = INFINITY;
  if (i < p.Nq) {
    const float l = p.lse[(int64_t)bh * p.Nq + i];
    l2 = l == -INFINITY ? INFINITY : l * kLog2e;
    const uint16_t* orow = p.o + (int64_t)b * p.o_s[0] + (int64_t)h * p.o_s[1] + (int64_t)i * p.o_s[2];
    const uint16_t* drow = p.dout + (int64_t)b * p.do_s[0] + (int64_t)h * p.do_s[1] + (int64_t)i * p.do_s[2];
    for (int d0 = 0; d0 < D; d0 += 8) {
      float xo[8], xd[8];
      unpack8<T>(ld16(orow + d0), xo);
      unpack8<T>(ld16(drow + d0), xd);
#pragma unroll
      for (int s = 0; s < 8; ++s) dl += xo[s] * xd[s];
    }
  }
  p.ld[idx] = make_float2(l2, dl);
}

// ---------------------------------------------------------------------------
template <int EP, int DV>
struct BwdCfg {
  static constexpr bool kBig = EP + DV > 160;
  static constexpr int BMK = kBig ? 32 : 64;   // query tile of a dK/dV job
  static constexpr int BNQ = kBig ? 32 : 64;   // key tile of a dQ job
  static constexpr int MINB = kBig ? 1 : 2;
  // Q_hat / dO (dK/dV jobs) and K_hat (dQ jobs) are read by rows and transposed: swizzled
  // strides; V (dQ jobs) only by rows.
  static constexpr int QH = 8 * lds_units_tr(EP / 8), DO = 8 * lds_units_tr(DV / 8);
  static constexpr int VR = 8 * lds_units_rows(DV / 8);
  // dK/dV stage: Q_hat tile, dO tile, lse and delta
  static constexpr int KV_STAGE = (BMK * QH + BMK * DO) * 2 + BMK * 8;
  // dQ stage: K_hat tile, V tile
  static constexpr int Q_STAGE = (BNQ * QH + BNQ * VR) * 2;
  static constexpr int STAGE = KV_STAGE > Q_STAGE ? KV_STAGE : Q_STAGE;
  static constexpr int EPI = 32 * (EP + 1) * 4;
  static constexpr int LDS = 2 * STAGE > EPI ? 2 * STAGE : EPI;
};

// dK / dV job.  Lane lr of wave w owns key j0 + 32 w + lr.
//   S  = Q_hat K_hat^T : A = Q_hat tile rows (LDS), B = the lane's K_hat row (regs)
//   dP = dO V^T        : A = dO tile rows (LDS),    B = the lane's V row (regs)
// Both results have lane = key, registers = queries, so P and dS are A operands
// (lane = key row, k = queries) of
//   dV     += P^T dO      B = dO tile read transposed
//   dK_hat += dS^T Q_hat  B = Q_hat tile read transposed
template <typename T, int EP, int DV>
__device__ __forceinline__ void dkdv_job(const FlashBwdParams& p, char* smem, float* dbias_s, int kb, int bhk) {
  typedef BwdCfg<EP, DV> C;
  constexpr int BM = C::BMK, KS = EP / 16, DS = DV / 16, EB = EP / 32, DB = DV / 32, QB = BM / 32;
  constexpr int QH = C::QH, DO = C::DO;
  constexpr int QCH = BM * (EP / 8), DCH = BM * (DV / 8);
  constexpr int QLD = (QCH + kThreads - 1) / kThreads, DLD = (DCH + kThreads - 1) / kThreads;
  typedef typename T::vec8 vec8;

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int b = bhk / p.Hk, hk = bhk % p.Hk;
  const int D = p.D, R = p.R, Nq = p.Nq, Nk = p.Nk, NqP = p.NqP;
  const int j0 = kb * 128;
  const int kj = j0 + 32 * wave + lr;

  const uint8_t* mrow = p.has_mask ? p.mask + (int64_t)b * p.mask_sb : nullptr;
  const bool kvis = kj < Nk && (!p.has_mask || mrow[kj] != 0);
  const TrLane dotr = tr_lane<true>(DO, lane), qhtr = tr_lane<true>(QH, lane);
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
  const float masked = -INFINITY;
  const int any_key = __syncthreads_or(kvis ? 1 : 0);
  const int nqt = (Nq + BM - 1) / BM;
  const int qt0 = p.causal ? min(j0 / BM, nqt) : 0;
  const int groups = p.Hq / p.Hk;
  const int per_head = nqt - qt0;
  const int nsteps = any_key ? groups * per_head : 0;

  // staging of one query tile: global -> registers -> LDS.  The fetch cursor (fg, fqt) walks
  // the group heads and query tiles in step order; pointers are per-job bases plus offsets.
  u32x4 qpf[QLD], dpf[DLD];
  float2 ldpf = make_float2(0.f, 0.f);
  const uint16_t* qh_job = p.qh + (int64_t)(b * p.Hq + hk) * NqP * EP;
  const int64_t qh_hstride = (int64_t)p.Hk * NqP * EP;
  const uint16_t* do_job = p.dout + (int64_t)b * p.do_s[0] + (int64_t)hk * p.do_s[1];
  const int64_t do_hstride = (int64_t)p.Hk * p.do_s[1];
  const int do_rs = (int)p.do_s[2];
  const float2* ld_job = p.ld + (int64_t)(b * p.Hq + hk) * NqP;
  const int64_t ld_hstride = (int64_t)p.Hk * NqP;
  int fg = 0, fqt = qt0;
  auto fetch = [&]() {
    const int i0 = fqt * BM;
    const uint16_t* qh_g = qh_job + fg * qh_hstride + (int64_t)i0 * EP;
    const uint16_t* do_g = do_job + fg * do_hstride;
    // Branch-free: chunk counts are whole multiples of the thread count where possible; rows
    // past Nq clamp to the last row (their P is 0: lse = +inf) and dims past D to the last
    // chunk (those columns only meet zero V columns, and their dV is never stored).
#pragma unroll
    for (int m = 0; m < QLD; ++m) {
      const int c = tid + m * kThreads;
      if (QCH % kThreads == 0 || c < QCH) qpf[m] = ld16(qh_g + (c / (EP / 8)) * EP + 8 * (c % (EP / 8)));
    }
#pragma unroll
    for (int m = 0; m < DLD; ++m) {
      const int c = tid + m * kThreads;
      if (DCH % kThreads == 0 || c < DCH) {
        const int row = min(i0 + c / (DV / 8), Nq - 1), d8 = min(8 * (c % (DV / 8)), D - 8);
        dpf[m] = ld16(do_g + (int64_t)row * do_rs + d8);
      }
    }
    if (tid < BM) ldpf = ld_job[fg * ld_hstride + i0 + tid];
    if (++fqt == nqt) {
      fqt = qt0;
      ++fg;
    }
  };
  auto stage = [&](int buf) {
    uint16_t* qh_s = reinterpret_cast<uint16_t*>(smem + buf * C::STAGE);
    uint16_t* do_s = qh_s + BM * QH;
    float2* ld_s = reinterpret_cast<float2*>(do_s + BM * DO);
#pragma unroll
    for (int m = 0; m < QLD; ++m) {
      const int c = tid + m * kThreads;
      const int row = c / (EP / 8);
      if (QCH % kThreads == 0 || c < QCH) st16(qh_s + row * QH + 8 * lds_swz(row, c % (EP / 8)), qpf[m]);
    }
#pragma unroll
    for (int m = 0; m < DLD; ++m) {
      const int c = tid + m * kThreads;
      const int row = c / (DV / 8);
      if (DCH % kThreads == 0 || c < DCH) st16(do_s + row * DO + 8 * lds_swz(row, c % (DV / 8)), dpf[m]);
    }
    if (tid < BM) ld_s[tid] = ldpf;
  };

  if (nsteps > 0) {
    fetch();
    stage(0);
  }
  __syncthreads();
  int i0 = qt0 * BM;   // query tile of the current step
  for (int st = 0; st < nsteps; ++st) {
    const int buf = st & 1;
    if (st + 1 < nsteps) fetch();
    const uint16_t* qh_s = reinterpret_cast<const uint16_t*>(smem + buf * C::STAGE);
    const uint16_t* do_s = qh_s + BM * QH;
    const float2* ld_s = reinterpret_cast<const float2*>(do_s + BM * DO);
#pragma unroll
    for (int qs = 0; qs < QB; ++qs) {
      f32x16 s = {}, dp = {};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        s = T::mfma32(as_vec8<vec8>(ld16(qh_s + (32 * qs + lr) * QH + 8 * lds_swz(lr, 2 * kk + hf))), kreg[kk], s);
#pragma unroll
      for (int kk = 0; kk < DS; ++kk)
        dp = T::mfma32(as_vec8<vec8>(ld16(do_s + (32 * qs + lr) * DO + 8 * lds_swz(lr, 2 * kk + hf))), vreg[kk], dp);
      // Partial sub-tile (some key of the wave masked, or on the causal diagonal): masked
      // scores become -inf so that P = 0.  Rows past Nq and fully
      // masked rows carry lse = +inf, which gives P = 0 without a test.
      if (!wave_vis || (p.causal && i0 + 32 * qs < j0 + 32 * wave + 31)) {
        POPE_COLD_PATH();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qr = 32 * qs + 8 * (r >> 2) + 4 * hf + (r & 3);
          s[r] = (kvis && (!p.causal || kj <= i0 + qr)) ? s[r] : masked;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qr = 32 * qs + 8 * (r >> 2) + 4 * hf + (r & 3);
        const float2 ld = ld_s[qr];
        const float pv = __builtin_amdgcn_exp2f(s[r] - ld.x);
        s[r] = pv;
        dp[r] = pv * (dp[r] - ld.y);
      }
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const vec8 ap = as_vec8<vec8>(pack8<T>(s, g2));
        const vec8 ads = as_vec8<vec8>(pack8<T>(dp, g2));
        const int r0 = 32 * qs + 16 * g2;
#pragma unroll
        for (int db = 0; db < DB; ++db)
          dva[db] = T::mfma32(ap, as_vec8<vec8>(lds_operand_tr(do_s, dotr, DO, r0, 32 * db)), dva[db]);
#pragma unroll
        for (int eb = 0; eb < EB; ++eb)
          dka[eb] = T::mfma32(ads, as_vec8<vec8>(lds_operand_tr(qh_s, qhtr, QH, r0, 32 * eb)), dka[eb]);
      }
    }
    if (st + 1 < nsteps) stage(buf ^ 1);
    __syncthreads();
    i0 = i0 + BM == nqt * BM ? qt0 * BM : i0 + BM;
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
  constexpr int BS = EP + 1;
  float* ebuf = reinterpret_cast<float*>(smem);
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
        if (dfb) atomicAdd(dfb + (int64_t)key * p.df_s[2] + d, dpsi);
        if (p.dbias) atomicAdd(&dbias_s[d], dpsi);
      } else {
        g = row[R + d] * kLn2;
      }
      dkb[(int64_t)key * p.dk_s[2] + d] = T::bits(g);
    }
  }
  if (p.dbias) {
    __syncthreads();
    for (int d = tid; d < R; d += kThreads) atomicAdd(p.dbias + (int64_t)hk * p.bias_sh + d, dbias_s[d]);
  }
}

// dQ job.  Lane lr of wave w owns query i0 + 32 w + lr.
//   S^T  = K_hat Q_hat^T : A = K_hat tile rows (LDS), B = the lane's Q_hat row (regs)
//   dP^T = V dO^T        : A = V tile rows (LDS),     B = the lane's dO row (regs)
// Results: lane = query, registers = keys; dS^T is the B operand of
//   dQ_hat^T += K_hat^T dS^T   A = K_hat tile read transposed.
template <typename T, int EP, int DV>
__device__ __forceinline__ void dq_job(const FlashBwdParams& p, char* smem, uint64_t* mbits_s, int qb, int bh) {
  typedef BwdCfg<EP, DV> C;
  constexpr int BN = C::BNQ, KS = EP / 16, DS = DV / 16, EB = EP / 32, NB = BN / 32;
  constexpr int KH = C::QH, VR = C::VR;
  constexpr int KCH = BN * (EP / 8), VCH = BN * (DV / 8);
  constexpr int KLD = (KCH + kThreads - 1) / kThreads, VLD = (VCH + kThreads - 1) / kThreads;
  typedef typename T::vec8 vec8;

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int bhk = b * p.Hk + hk;
  const int D = p.D, R = p.R, Nq = p.Nq, Nk = p.Nk, NkP = p.NkP;
  const int q_off = Nk - Nq;
  const int qi = qb * 128 + 32 * wave + lr;
  const bool qvalid = qi < Nq;
  const TrLane khtr = tr_lane<true>(KH, lane);

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
  const float masked = -INFINITY;
  const float2 ld = p.ld[(int64_t)bh * p.NqP + qi];   // rows past Nq: lse = +inf
  const float lse2 = ld.x, dl = ld.y;

  f32x16 dqa[EB];
#pragma unroll
  for (int x = 0; x < EB; ++x)
#pragma unroll
    for (int r = 0; r < 16; ++r) dqa[x][r] = 0.f;

  int nt = (Nk + BN - 1) / BN;
  if (p.causal) {
    const int last_q = min(qb * 128 + 128, Nq) - 1;
    nt = last_q < 0 ? 0 : min(nt, last_q / BN + 1);
  }
  const uint16_t* kh_g = p.kh + (int64_t)bhk * NkP * EP;
  const uint16_t* v_g = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  const uint8_t* mrow = p.has_mask ? p.mask + (int64_t)b * p.mask_sb : nullptr;

  u32x4 kpf[KLD], vpf[VLD];
  uint64_t mpf = 0;
  auto fetch = [&](int kt) {
    const int j0 = kt * BN;
    // Branch-free as in the dK/dV job: keys past Nk clamp to the last row (masked, P = 0) and
    // dims past D to the last chunk (those columns only meet zero dO columns).
#pragma unroll
    for (int m = 0; m < KLD; ++m) {
      const int c = tid + m * kThreads;
      if (KCH % kThreads == 0 || c < KCH) kpf[m] = ld16(kh_g + (int64_t)(j0 + c / (EP / 8)) * EP + 8 * (c % (EP / 8)));
    }
#pragma unroll
    for (int m = 0; m < VLD; ++m) {
      const int c = tid + m * kThreads;
      if (VCH % kThreads == 0 || c < VCH) {
        const int row = min(j0 + c / (DV / 8), Nk - 1), d8 = min(8 * (c % (DV / 8)), D - 8);
        vpf[m] = ld16(v_g + (int64_t)row * p.v_s[2] + d8);
      }
    }
    if (wave == 0) {   // bit j: key j0 + j visible
      const int key = j0 + lane;
      mpf = __ballot(lane < BN && key < Nk && (!p.has_mask || mrow[key] != 0));
    }
  };
  auto stage = [&](int buf) {
    uint16_t* kh_s = reinterpret_cast<uint16_t*>(smem + buf * C::STAGE);
    uint16_t* v_s = kh_s + BN * KH;
#pragma unroll
    for (int m = 0; m < KLD; ++m) {
      const int c = tid + m * kThreads;
      const int row = c / (EP / 8);
      if (KCH % kThreads == 0 || c < KCH) st16(kh_s + row * KH + 8 * lds_swz(row, c % (EP / 8)), kpf[m]);
    }
#pragma unroll
    for (int m = 0; m < VLD; ++m) {
      const int c = tid + m * kThreads;
      if (VCH % kThreads == 0 || c < VCH) st16(v_s + (c / (DV / 8)) * VR + 8 * (c % (DV / 8)), vpf[m]);
    }
    if (tid == 0) mbits_s[buf] = mpf;
  };

  if (nt > 0) {
    fetch(0);
    stage(0);
  }
  __syncthreads();
  for (int kt = 0; kt < nt; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nt) fetch(kt + 1);
    const int j0 = kt * BN;
    const uint16_t* kh_s = reinterpret_cast<const uint16_t*>(smem + buf * C::STAGE);
    const uint16_t* v_s = kh_s + BN * KH;
    const uint64_t mraw = mbits_s[buf];
    const uint64_t mb = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)mraw) |
                        ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(mraw >> 32)) << 32);
    const uint64_t all_bits = BN == 64 ? ~0ull : ((1ull << BN) - 1);
    // every key visible and (causal) every key at or before the wave's first query
    const bool full = mb == all_bits && !(p.causal && j0 + BN - 1 > qb * 128 + 32 * wave);
    if (mb == 0) {   // every key of this tile masked
      if (kt + 1 < nt) stage(buf ^ 1);
      __syncthreads();
      continue;
    }
#pragma unroll
    for (int ks = 0; ks < NB; ++ks) {
      f32x16 s = {}, dp = {};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        s = T::mfma32(as_vec8<vec8>(ld16(kh_s + (32 * ks + lr) * KH + 8 * lds_swz(lr, 2 * kk + hf))), qreg[kk], s);
#pragma unroll
      for (int kk = 0; kk < DS; ++kk)
        dp = T::mfma32(as_vec8<vec8>(ld16(v_s + (32 * ks + lr) * VR + 16 * kk + 8 * hf)), doreg[kk], dp);
      if (!full) {   // masked scores -> -inf: P = 0
        POPE_COLD_PATH();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kr = 32 * ks + 8 * (r >> 2) + 4 * hf + (r & 3);
          s[r] = (((mb >> kr) & 1ull) && (!p.causal || j0 + kr <= qi)) ? s[r] : masked;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] = __builtin_amdgcn_exp2f(s[r] - lse2) * (dp[r] - dl);
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const vec8 bds = as_vec8<vec8>(pack8<T>(dp, g2));
#pragma unroll
        for (int eb = 0; eb < EB; ++eb)
          dqa[eb] = T::mfma32(as_vec8<vec8>(lds_operand_tr(kh_s, khtr, KH, 32 * ks + 16 * g2, 32 * eb)), bds, dqa[eb]);
      }
    }
    if (kt + 1 < nt) stage(buf ^ 1);
    __syncthreads();
  }

  // ---- dQ: query-side chain rule, one wave's 32 queries at a time through LDS ----
  constexpr int BS = EP + 1;
  float* ebuf = reinterpret_cast<float*>(smem);
  const uint16_t* qb_ptr = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1];
  uint16_t* dqb = p.dq + (int64_t)b * p.dq_s[0] + (int64_t)h * p.dq_s[1];
  const float2* tq = R ? p.table + (int64_t)b * p.t_sb + (int64_t)h * p.t_sh : nullptr;
  const float2* bq = R ? p.btab + (p.Hb > 1 ? hk : 0) * R : nullptr;
  float* dfb = p.dfreqs ? p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)h * p.df_s[1] : nullptr;
  for (int w = 0; w < 4; ++w) {
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
      const int i = qb * 128 + 32 * w + qr;
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
        if (dfb) atomicAdd(dfb + (int64_t)(q_off + i) * p.df_s[2] + d, softplus_f(x) * (cs * us - sn * uc));
      } else {
        g = row[R + d] * p.scale;
      }
      dqb[(int64_t)i * p.dq_s[2] + d] = T::bits(g);
    }
  }
}

template <typename T, int EP, int DV>
__global__ __launch_bounds__(kThreads, (BwdCfg<EP, DV>::MINB)) void bwd_main_kernel(FlashBwdParams p) {
  __shared__ __attribute__((aligned(16))) char smem[BwdCfg<EP, DV>::LDS];
  __shared__ float dbias_s[EP];
  __shared__ uint64_t mbits_s[2];
  const int nqb = p.NqP / 128;
  const int id = blockIdx.x;
  int kind, blk, head;   // kind 0 = dK/dV job (head = b * Hk + hk), 1 = dQ job (head = b * Hq + h)
  if (p.interleave) {
    // pairs of equal cost, heaviest first: dK/dV block r with dQ block nqb - 1 - r; the
    // batch * head index is fastest so that one head's jobs share an XCD (workgroup ids are
    // dealt round-robin over the 8 XCDs)
    const int BH = p.B * p.Hq;
    const int r = id / (2 * BH), rem = id % (2 * BH);
    kind = rem / BH;
    head = rem % BH;
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
    dq_job<T, EP, DV>(p, smem, mbits_s, blk, head);
}

template <typename T, int EP, int DV>
hipError_t launch_t(const FlashBwdParams& p0, hipStream_t s) {
  FlashBwdParams p = p0;
  const int64_t nrows = (int64_t)p.B * p.Hq * p.NqP;
  hipError_t e = launch_named("flash_bwd_delta", bwd_delta_kernel<T>, dim3((unsigned)((nrows + 255) / 256)),
                              dim3(256), s, p);
  if (e != hipSuccess) return e;
  const int nkb = p.NkP / 128, nqb = p.NqP / 128;
  p.n_kv_jobs = nkb * p.B * p.Hk;
  p.interleave = p.causal && p.Hq == p.Hk && nkb == nqb && p.Nq == p.Nk;
  const int jobs = p.n_kv_jobs + nqb * p.B * p.Hq;
  return launch_named("flash_bwd", bwd_main_kernel<T, EP, DV>, dim3(jobs), dim3(kThreads), s, p);
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
