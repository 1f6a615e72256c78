// Flash attention with PoPE for wide heads: head dims of 136 to 256 (after padding to a multiple
// of 8), expanded rows up to 512 features (gfx950, bf16 / fp16 MFMA).
//
// Reference semantics: triton_pope_flash_attn.py:23-117 (forward), :119-218 (backward), whose
// Triton kernels take any head dim (BD = next_pow2(D), :252-254); PyTorch path
// attention.py:106-145.
//
// The rows of these heads do not fit the register tiling of flash_fwd.hip / flash_bwd.hip (the
// backward's dK_hat accumulator alone is 256 registers per lane at E = 512), so the wide path
// trades speed for a plain structure: four waves per workgroup (one per SIMD, up to 512
// registers), 32 rows per wave, the backward's accumulators split into as few column chunks as the
// registers allow (each chunk recomputes the scores; the other waves take neighbouring row blocks),
// tiles shared by the four waves through LDS, and the polar transform's chain rule in a separate
// pass.  The streamed tiles go straight from global memory into LDS (global_load_lds_dwordx4) in
// three slots, two steps ahead of the step computed: a step's products take less time than the
// tile's fetch, and tiles staged through registers would hold registers these kernels do not
// have.  Memory stays linear in the sequence length: no score matrix is stored.  Same workspace preparation as the narrow path
// (flash_prep.hip: K_hat, Q_hat pre-scaled by softmax_scale * log2 e, key visibility words,
// phase tables), with EP = E rounded up to 128 and DV = 256.
//   wide_fwd   one workgroup per (128 queries, batch * head): S^T = K_hat Q_hat^T, online softmax
//              in log2 units, O^T += V^T P^T with V read transposed (ds_read_b64_tr_b16); the
//              K_hat and V tiles of 32 keys streamed through LDS.
//   wide_kv    one workgroup per (key blocks, batch * kv head), wave = (32 keys, column chunk): S = Q_hat K_hat^T
//              - lse, dP = dO V^T - delta (Q_hat and dO tiles and the row terms streamed through
//              LDS), P = exp2 S,
//              dS = P dP; dV (the wave's chunk of D columns) += P^T dO and dK_hat (its chunk of E
//              columns) += dS^T Q_hat; writes dV and the raw dK_hat chunk (fp32 workspace).
//   wide_q     one workgroup per (query blocks, batch * head), wave = (32 queries, column chunk): S^T, dP^T with
//              the K_hat and V tiles in LDS, dQ_hat^T (its chunk) += K_hat^T dS^T; writes the raw
//              dQ_hat chunk.
//   wide_chain the chain rule of the polar transform from the raw rows: dk, dq, dfreqs, dbias
//              (deterministic mode: the per-row phase derivatives, summed later in a fixed order).
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {


__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

typedef const __attribute__((address_space(4))) uint64_t cu64;
typedef const __attribute__((address_space(4))) int ci32;

// Registers [8 g, 8 g + 8) of an MFMA result, packed as an 8-element operand.
template <typename T>
__device__ __forceinline__ u32x4 pack8w(const f32x16& x, int g) {
  u32x4 w;
#pragma unroll
  for (int s = 0; s < 4; ++s) w[s] = T::pack2(x[8 * g + 2 * s], x[8 * g + 2 * s + 1]);
  return w;
}

__device__ __forceinline__ f32x16 splat16(float x) {
  f32x16 c;
#pragma unroll
  for (int r = 0; r < 16; ++r) c[r] = x;
  return c;
}

// Row offset within a 32-row block of register r of a 32x32 MFMA result in lane half hf.
__device__ __forceinline__ int res_row(int r, int hf) { return 8 * (r >> 2) + 4 * hf + (r & 3); }

// Growth of a row's running max (log2 units) that the forward absorbs without rescaling its
// accumulators: probabilities reach at most 2^kLazyMax.
constexpr float kLazyMax = 8.f;

// LDS slots of the streamed tiles: tile t is computed from slot t % kSlots while tiles t + 1 and
// t + 2 load, so each tile has two steps of compute to arrive in.
constexpr int kSlots = 3;

// Transpose-read offsets (lo, hi) of column block nb of a tile, nb known only at run time: the
// entry of the swizzle period is picked by selects rather than by indexing the offset arrays,
// which would place them in scratch memory (vector loads that would wait on the tile loads).
template <int U>
__device__ __forceinline__ int2 tr_offsets(const TileOffsets<U>& o, int nb) {
  constexpr int TP = TileOffsets<U>::TP;
  const int k = nb % TP;
  int lo = o.lo[0], hi = o.hi[0];
#pragma unroll
  for (int i = 1; i < TP; ++i) {
    lo = k == i ? o.lo[i] : lo;
    hi = k == i ? o.hi[i] : hi;
  }
  return make_int2(lo + 32 * (nb - k), hi + 32 * (nb - k));
}

// Direct global -> LDS fill of one tile of 32 rows x U 16-byte units, stored unpadded with
// tile_swz (unit u of row r at position u ^ tile_swz(U, r)).  Load i of the thread fills
// position c = 256 i + tid (a wave's 64 lanes write 64 consecutive positions), in row c / U,
// with unit (c % U) ^ tile_swz(U, c / U) of that row; src(r, u) is its global address.
template <int U, typename Src>
__device__ __forceinline__ void tile_fill(const uint16_t* tile, int tid, int wave, Src src) {
  static_assert(32 * U % 256 == 0, "whole loads per thread");
  const uint32_t base = lds_addr(tile) + 1024 * wave;
#pragma unroll
  for (int i = 0; i < 32 * U / 256; ++i) {
    const int c = tid + 256 * i, r = c / U;
    load_lds16(src(r, (c % U) ^ tile_swz(U, r)), base + 4096 * i);
  }
}

// ---- forward ---------------------------------------------------------------------------
// Four waves per workgroup, 128 query rows (wave w: rows q0 + 32 w ..); per 32-key tile the K_hat
// rows and the V rows go straight from global memory into LDS once for the four waves (unpadded,
// XOR-swizzled), in three slots: the loads of the next two tiles are in flight while the current
// tile is computed.
template <typename T, int EP, int DV>
__global__ __launch_bounds__(256) void wide_fwd_kernel(FlashFwdParams p) {
  constexpr int KS = EP / 16, NDB = DV / 32;
  constexpr int KU = EP / 8, VU = DV / 8;              // 16-byte units per K_hat / V row
  constexpr int NL = 32 * (KU + VU) / 256;             // loads per thread and tile
  typedef typename T::vec8 vec8;
  __shared__ __attribute__((aligned(16))) uint16_t kt[kSlots][32 * EP];
  __shared__ __attribute__((aligned(16))) uint16_t vt[kSlots][32 * DV];

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int BH = p.B * p.Hq, nqb = p.NqP / 128;
  const int bh = blockIdx.x % BH;
  const int q0 = 128 * (nqb - 1 - (int)(blockIdx.x / BH));   // heaviest causal blocks first
  if (q0 >= p.Nq) return;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int Nk = p.Nk, D = p.D, qi = q0 + 32 * wave + lr;

  int nkeys = min(((ci32*)p.kend)[b], Nk);
  if (p.causal) nkeys = min(nkeys, q0 + 128);
  const uint16_t* khb = p.kh + (int64_t)(b * p.Hk + hk) * p.NkP * EP;   // rows padded to NkP
  const uint16_t* vb = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  cu64* mw = (cu64*)p.mwords + (int64_t)b * p.NW;
  const TileOffsets<KU> ko(lane);
  const TileOffsets<VU> vo(lane);

  // tile t into slot t % kSlots: K_hat rows are padded to NkP (no clamp); V rows past Nk repeat
  // the last one and V units at or past D repeat the row's last unit (they only reach the O rows
  // at or past D, which are not stored)
  auto issue = [&](int t) {
    const int j0 = 32 * t, slot = t % kSlots;
    const uint16_t* kp = khb + (int64_t)j0 * EP;
    tile_fill<KU>(kt[slot], tid, wave, [&](int r, int u) { return kp + r * EP + 8 * u; });
    tile_fill<VU>(vt[slot], tid, wave, [&](int r, int u) {
      return vb + (int64_t)min(j0 + r, Nk - 1) * p.v_s[2] + min(8 * u, D - 8);
    });
  };
  const int nt = (nkeys + 31) / 32;
  if (nt > 0) issue(0);
  if (nt > 1) issue(1);

  vec8 qreg[KS];
  {
    const uint16_t* qrow = p.qh + ((int64_t)bh * p.NqP + qi) * EP + 8 * hf;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qreg[kk] = as_vec8<vec8>(ld16(qrow + 16 * kk));
  }
  // the Q_hat rows as loads the compiler sees complete: no use of them in the loop waits on the
  // tile loads in flight there
  settle_vector_loads();

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = splat16(0.f);
  float m = -INFINITY, l = 0.f;
  const uint32_t ones = T::pack2(1.f, 1.f);
  for (int t = 0; t < nt; ++t) {
    const int buf = t % kSlots, j0 = 32 * t;
    if (t + 1 < nt) wait_vmcnt<NL>();   // this thread's loads of tile t landed (t + 1 may be in flight)
    else wait_vmcnt<0>();
    __syncthreads();                    // ... everyone's; and slot (t + 2) % kSlots was last read in step t - 1
    if (t + 2 < nt) issue(t + 2);
    // S^T (rows = keys, lane = query), log2 units
    f32x16 s = splat16(0.f);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      s = T::mfma32(as_vec8<vec8>(*reinterpret_cast<const u32x4*>(kt[buf] + ko.row_at(kk))), qreg[kk], s);
    const uint32_t wv = (uint32_t)(mw[j0 >> 6] >> (j0 & 32));
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr_ = res_row(r, hf);
      const bool ok = ((wv >> kr_) & 1u) && (!p.causal || j0 + kr_ <= qi);
      s[r] = ok ? s[r] : -INFINITY;
      mt = fmaxf(mt, s[r]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    float alpha = 1.f;
    if constexpr (EP < 512) {
      // lazy rescale: a row's reference max m moves only when the tile's max exceeds it by more
      // than kLazyMax (log2 units), so the probabilities stay below 2^kLazyMax and most steps skip
      // rescaling the O accumulators (the branch is taken when any row of the wave moves).  At
      // 512 features the branch costs more than it saves: the rescale stays in every step.
      const bool grow = mt > m + kLazyMax;
      if (__ballot(grow)) {
        const float mn = grow ? mt : m;
        alpha = __builtin_amdgcn_exp2f(m - (mn == -INFINITY ? 0.f : mn));
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
        m = mn;   // l takes alpha below
      }
    } else {
      const float mn = fmaxf(m, mt);
      alpha = __builtin_amdgcn_exp2f(m - (mn == -INFINITY ? 0.f : mn));
      m = mn;
    }
    const float mu = m == -INFINITY ? 0.f : m;
    u32x4 pw[2];
    float ls = 0.f;
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w = T::pack2(__builtin_amdgcn_exp2f(s[8 * g + 2 * q] - mu),
                                    __builtin_amdgcn_exp2f(s[8 * g + 2 * q + 1] - mu));
        pw[g][q] = w;
        ls = T::dot2(w, ones, ls);   // the row sum of the probabilities the products use
      }
    l = l * alpha + ls + __shfl_xor(ls, 32, 64);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      if constexpr (EP >= 512) {
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
      }
#pragma unroll
      for (int g = 0; g < 2; ++g)
        oacc[db] = T::mfma32(as_vec8<vec8>(lds_tr8(vt[buf], vo.lo_at(db) + 16 * g * DV, vo.hi_at(db) + 16 * g * DV)),
                             as_vec8<vec8>(pw[g]), oacc[db]);
    }
  }
  if (qi >= p.Nq) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
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
    p.lse[((int64_t)b * p.Hq + h) * p.Nq + qi] = m == -INFINITY ? -INFINITY : (m + __builtin_amdgcn_logf(l)) * kLn2;
}

// ---- backward: dK_hat / dV --------------------------------------------------------------
// One workgroup per (4 / CH blocks of 32 keys, batch * kv head); wave w takes key block w / CH and
// column chunk w % CH of the accumulators (CH chunks recompute the scores CH times; fewer where the
// registers allow).  The Q_hat and dO tiles of each 32-query step go straight from global memory
// into LDS once for the four waves, in three slots (two steps ahead of the step computed), with
// the step's -lse and -delta rows (one more load, wave 0).
template <typename T, int EP, int DV, int CH>
__global__ __launch_bounds__(256) void wide_kv_kernel(FlashBwdParams p, float* wk) {
  constexpr int KS = EP / 16, DS = DV / 16, EBC = EP / 32 / CH, DBC = DV / 32 / CH, RB = 4 / CH;
  constexpr int QU = EP / 8, OU = DV / 8, NL = 32 * (QU + OU) / 256;
  typedef typename T::vec8 vec8;
  __shared__ __attribute__((aligned(16))) uint16_t qt[kSlots][32 * EP];
  __shared__ __attribute__((aligned(16))) uint16_t dt[kSlots][32 * DV];
  __shared__ __attribute__((aligned(16))) float rt[kSlots][256];   // [0, 32) -lse, [32, 64) -delta

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int nkb = p.NkP / (32 * RB);
  const int ec = (tid >> 6) % CH;   // the wave's column chunk
  const int kb0 = 32 * RB * ((int)blockIdx.x % nkb), bhk = (int)blockIdx.x / nkb;   // key block 0 (the heaviest causal one) first
  const int k0 = kb0 + 32 * ((tid >> 6) / CH);   // the wave's keys
  const int b = bhk / p.Hk, hk = bhk % p.Hk;
  const int Nk = p.Nk, Nq = p.Nq, D = p.D, NqP = p.NqP;
  if (kb0 >= Nk) return;
  const int kj = k0 + lr;
  cu64* mw = (cu64*)p.mwords + (int64_t)b * p.NW;
  const bool kvis = kj < Nk && ((mw[kj >> 6] >> (kj & 63)) & 1ull);

  // the steps: (query head g of the kv head's group, 32-query block q0), flattened
  const int groups = p.Hq / p.Hk;
  const int qstart = p.causal ? kb0 : 0;   // the workgroup's first key block
  const int nsq = Nq > qstart ? (Nq - qstart + 31) / 32 : 0;
  const int nsteps = __syncthreads_or(kvis) ? groups * nsq : 0;   // uniform over the workgroup
  auto step_at = [&](int st, int& h, int& q0) {
    h = (st / nsq) * p.Hk + hk;
    q0 = qstart + 32 * (st % nsq);
  };
  // step st's tiles into slot st % kSlots: Q_hat rows padded to NqP (no clamp); dO rows past Nq
  // repeat the last one and dO units at or past D repeat the row's last unit (they meet zero V
  // columns in dP and reach only the dV columns at or past D, which are not stored)
  auto issue = [&](int st) {
    int h, q0;
    step_at(st, h, q0);
    const int slot = st % kSlots;
    const uint16_t* qhb = p.qh + ((int64_t)(b * p.Hq + h) * NqP + q0) * EP;
    const uint16_t* dob = p.dout + (int64_t)b * p.do_s[0] + (int64_t)h * p.do_s[1];
    tile_fill<QU>(qt[slot], tid, wave, [&](int r, int u) { return qhb + r * EP + 8 * u; });
    tile_fill<OU>(dt[slot], tid, wave, [&](int r, int u) {
      return dob + (int64_t)min(q0 + r, Nq - 1) * p.do_s[2] + min(8 * u, D - 8);
    });
    // the row terms of queries q0 .. q0 + 31: lane units 0-7 -lse, 8-15 -delta (lanes past 15
    // repeat them past float 64, unread)
    if (wave == 0) {
      const int u = lane & 15;
      const float* src = (u < 8 ? p.nl : p.nd) + (int64_t)(b * p.Hq + h) * NqP + q0 + 4 * (u & 7);
      load_lds16(src, lds_addr(rt[slot]));
    }
  };
  if (nsteps > 0) issue(0);
  if (nsteps > 1) issue(1);

  vec8 kreg[KS], vreg[DS];
  {
    const uint16_t* khr = p.kh + ((int64_t)bhk * p.NkP + kj) * EP + 8 * hf;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) kreg[kk] = as_vec8<vec8>(ld16(khr + 16 * kk));
    const uint16_t* vr = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1] + (int64_t)min(kj, Nk - 1) * p.v_s[2];
#pragma unroll
    for (int kk = 0; kk < DS; ++kk) {
      const int d0 = 16 * kk + 8 * hf;
      vreg[kk] = as_vec8<vec8>((kj < Nk && d0 < D) ? ld16(vr + d0) : zero4());
    }
  }
  // the K_hat / V rows as loads the compiler sees complete: no use of them in the loop waits on
  // the tile loads in flight there
  settle_vector_loads();
  f32x16 dka[EBC], dva[DBC];
#pragma unroll
  for (int x = 0; x < EBC; ++x) dka[x] = splat16(0.f);
#pragma unroll
  for (int x = 0; x < DBC; ++x) dva[x] = splat16(0.f);
  // the tiles' row-read offsets, and the wave's transpose-read offsets: its dV column blocks of
  // the dO tile, its dK_hat column blocks of the Q_hat tile
  const TileOffsets<QU> qo(lane);
  const TileOffsets<OU> dO(lane);
  int2 dof[DBC], qof[EBC];
#pragma unroll
  for (int db = 0; db < DBC; ++db) dof[db] = tr_offsets(dO, ec * DBC + db);
#pragma unroll
  for (int eb = 0; eb < EBC; ++eb) qof[eb] = tr_offsets(qo, ec * EBC + eb);

  for (int st = 0; st < nsteps; ++st) {
    const int buf = st % kSlots;
    int h, q0;
    step_at(st, h, q0);
    // this thread's loads of step st landed (st + 1 may be in flight; wave 0 has one more per step)
    if (st + 1 < nsteps) {
      if (wave == 0) wait_vmcnt<NL + 1>();
      else wait_vmcnt<NL>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();                         // ... everyone's; and slot (st + 2) % kSlots was last read in step st - 1
    if (st + 2 < nsteps) issue(st + 2);
    // -lse and -delta of the result rows (queries q0 + res_row(r, hf); padded rows give P = 0)
    f32x16 s, dp;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(&rt[buf][8 * q + 4 * hf]);
      const f32x4 c = *reinterpret_cast<const f32x4*>(&rt[buf][32 + 8 * q + 4 * hf]);
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        s[4 * q + x] = a[x];
        dp[4 * q + x] = c[x];
      }
    }
    // S = Q_hat K_hat^T - lse and dP = dO V^T - delta (rows = queries, lane = key)
#pragma unroll
    for (int kg = 0; kg < KS; kg += 8) {
#pragma unroll
      for (int kk = kg; kk < kg + 8; ++kk)
        s = T::mfma32(as_vec8<vec8>(*reinterpret_cast<const u32x4*>(qt[buf] + qo.row_at(kk))), kreg[kk], s);
      __builtin_amdgcn_sched_barrier(0);   // eight operand reads in flight, not all of them
    }
#pragma unroll
    for (int kg = 0; kg < DS; kg += 8) {
#pragma unroll
      for (int kk = kg; kk < kg + 8; ++kk)
        dp = T::mfma32(as_vec8<vec8>(*reinterpret_cast<const u32x4*>(dt[buf] + dO.row_at(kk))), vreg[kk], dp);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool ok = kvis && (!p.causal || kj <= q0 + res_row(r, hf));
      const float pv = ok ? __builtin_amdgcn_exp2f(s[r]) : 0.f;
      s[r] = pv;
      dp[r] = pv * dp[r];
    }
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      const vec8 ap = as_vec8<vec8>(pack8w<T>(s, g2)), ads = as_vec8<vec8>(pack8w<T>(dp, g2));
#pragma unroll
      for (int db = 0; db < DBC; ++db)
        dva[db] = T::mfma32(
            ap, as_vec8<vec8>(lds_tr8(dt[buf], dof[db].x + 16 * g2 * DV, dof[db].y + 16 * g2 * DV)), dva[db]);
#pragma unroll
      for (int eb = 0; eb < EBC; ++eb)
        dka[eb] = T::mfma32(
            ads, as_vec8<vec8>(lds_tr8(qt[buf], qof[eb].x + 16 * g2 * EP, qof[eb].y + 16 * g2 * EP)), dka[eb]);
    }
  }
  // dV (lane = d column, registers = keys); the raw dK_hat chunk, times ln 2 (Q_hat carries log2 e)
  uint16_t* dvb = p.dv + (int64_t)b * p.dv_s[0] + (int64_t)hk * p.dv_s[1];
#pragma unroll
  for (int db = 0; db < DBC; ++db) {
    const int d = 32 * (ec * DBC + db) + lr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + res_row(r, hf);
      if (key < Nk && d < D) dvb[(int64_t)key * p.dv_s[2] + d] = T::bits(dva[db][r]);
    }
  }
  float* wkb = wk + (int64_t)bhk * p.NkP * EP;
#pragma unroll
  for (int eb = 0; eb < EBC; ++eb) {
    const int e = 32 * (ec * EBC + eb) + lr;
#pragma unroll
    for (int r = 0; r < 16; ++r) wkb[(int64_t)(k0 + res_row(r, hf)) * EP + e] = dka[eb][r] * kLn2;
  }
}

// ---- backward: dQ_hat -------------------------------------------------------------------
// One workgroup per (4 / CH blocks of 32 queries, batch * head); wave w takes query block w / CH
// and column chunk w % CH of the accumulator.  The K_hat and V tiles of each 32-key step go
// straight from global memory into LDS once for the four waves, in three slots (two steps ahead).
template <typename T, int EP, int DV, int CH>
__global__ __launch_bounds__(256) void wide_q_kernel(FlashBwdParams p, float* wq) {
  constexpr int KS = EP / 16, DS = DV / 16, EBC = EP / 32 / CH, RB = 4 / CH;
  constexpr int KU = EP / 8, VU = DV / 8, NL = 32 * (KU + VU) / 256;
  typedef typename T::vec8 vec8;
  __shared__ __attribute__((aligned(16))) uint16_t kt[kSlots][32 * EP];
  __shared__ __attribute__((aligned(16))) uint16_t vt[kSlots][32 * DV];

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int nqb = p.NqP / (32 * RB);
  const int ec = (tid >> 6) % CH;   // the wave's column chunk
  const int qb0 = 32 * RB * (nqb - 1 - (int)blockIdx.x % nqb), bh = (int)blockIdx.x / nqb;   // heaviest causal blocks first
  const int q0 = qb0 + 32 * ((tid >> 6) / CH);   // the wave's queries
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int Nk = p.Nk, Nq = p.Nq, D = p.D;
  if (qb0 >= Nq) return;
  const int qi = q0 + lr;
  int nkeys = min(((ci32*)p.kend)[b], Nk);
  if (p.causal) nkeys = min(nkeys, qb0 + 32 * RB);   // the workgroup's last query block
  const uint16_t* khb = p.kh + (int64_t)(b * p.Hk + hk) * p.NkP * EP;   // rows padded to NkP
  const uint16_t* vb = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  // tile t into slot t % kSlots: K_hat rows padded to NkP (no clamp); V rows past Nk repeat the
  // last one and V units at or past D repeat the row's last unit (they meet zero dO columns)
  auto issue = [&](int t) {
    const int j0 = 32 * t, slot = t % kSlots;
    const uint16_t* kp = khb + (int64_t)j0 * EP;
    tile_fill<KU>(kt[slot], tid, wave, [&](int r, int u) { return kp + r * EP + 8 * u; });
    tile_fill<VU>(vt[slot], tid, wave, [&](int r, int u) {
      return vb + (int64_t)min(j0 + r, Nk - 1) * p.v_s[2] + min(8 * u, D - 8);
    });
  };
  const int nt = (nkeys + 31) / 32;
  if (nt > 0) issue(0);
  if (nt > 1) issue(1);

  vec8 qreg[KS], doreg[DS];
  {
    const uint16_t* qhr = p.qh + ((int64_t)bh * p.NqP + qi) * EP + 8 * hf;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qreg[kk] = as_vec8<vec8>(ld16(qhr + 16 * kk));
    const uint16_t* dr = p.dout + (int64_t)b * p.do_s[0] + (int64_t)h * p.do_s[1] + (int64_t)min(qi, Nq - 1) * p.do_s[2];
#pragma unroll
    for (int kk = 0; kk < DS; ++kk) {
      const int d0 = 16 * kk + 8 * hf;
      doreg[kk] = as_vec8<vec8>((qi < Nq && d0 < D) ? ld16(dr + d0) : zero4());
    }
  }
  const float nls = p.nl[(int64_t)bh * p.NqP + qi], nds = p.nd[(int64_t)bh * p.NqP + qi];
  // the row loads as loads the compiler sees complete: no use of them in the loop waits on the
  // tile loads in flight there
  settle_vector_loads();
  f32x16 dqa[EBC];
#pragma unroll
  for (int x = 0; x < EBC; ++x) dqa[x] = splat16(0.f);
  cu64* mw = (cu64*)p.mwords + (int64_t)b * p.NW;
  const TileOffsets<KU> ko(lane);
  const TileOffsets<VU> vo(lane);
  for (int t = 0; t < nt; ++t) {
    const int buf = t % kSlots, j0 = 32 * t;
    if (t + 1 < nt) wait_vmcnt<NL>();   // this thread's loads of tile t landed (t + 1 may be in flight)
    else wait_vmcnt<0>();
    __syncthreads();                    // ... everyone's; and slot (t + 2) % kSlots was last read in step t - 1
    if (t + 2 < nt) issue(t + 2);
    // S^T = K_hat Q_hat^T - lse and dP^T = V dO^T - delta (rows = keys, lane = query)
    f32x16 s = splat16(nls), dp = splat16(nds);
#pragma unroll
    for (int kg = 0; kg < KS; kg += 8) {
#pragma unroll
      for (int kk = kg; kk < kg + 8; ++kk)
        s = T::mfma32(as_vec8<vec8>(*reinterpret_cast<const u32x4*>(kt[buf] + ko.row_at(kk))), qreg[kk], s);
      __builtin_amdgcn_sched_barrier(0);   // eight operand reads in flight, not all of them
    }
#pragma unroll
    for (int kg = 0; kg < DS; kg += 8) {
#pragma unroll
      for (int kk = kg; kk < kg + 8; ++kk)
        dp = T::mfma32(as_vec8<vec8>(*reinterpret_cast<const u32x4*>(vt[buf] + vo.row_at(kk))), doreg[kk], dp);
      __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t wv = (uint32_t)(mw[j0 >> 6] >> (j0 & 32));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr_ = res_row(r, hf);
      const bool ok = ((wv >> kr_) & 1u) && (!p.causal || j0 + kr_ <= qi);
      dp[r] = ok ? __builtin_amdgcn_exp2f(s[r]) * dp[r] : 0.f;
    }
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      const vec8 bds = as_vec8<vec8>(pack8w<T>(dp, g2));
#pragma unroll
      for (int eb = 0; eb < EBC; ++eb)
        dqa[eb] = T::mfma32(
            as_vec8<vec8>(lds_tr8(kt[buf], ko.lo_at(ec * EBC + eb) + 16 * g2 * EP, ko.hi_at(ec * EBC + eb) + 16 * g2 * EP)),
            bds, dqa[eb]);
    }
  }
  // the raw dQ_hat chunk (rows = e, lane = query), times softmax_scale
  float* wqb = wq + ((int64_t)bh * p.NqP + qi) * EP;
#pragma unroll
  for (int eb = 0; eb < EBC; ++eb)
#pragma unroll
    for (int r = 0; r < 16; ++r) wqb[32 * (ec * EBC + eb) + res_row(r, hf)] = dqa[eb][r] * p.scale;
}

// ---- the chain rule of the polar transform -----------------------------------------------
// Blocks [0, nk): 32 key rows of one (batch, kv head); blocks [nk, nk + nq): 32 query rows of
// one (batch, head).  With the raw expanded-row gradients U (cos column e = d, sin column
// e = R + d, pass-through column e = R + d) and the row's phase (keys F[j]; queries
// F[q_off + i] - bias, the bias on the query side as in the preparation):
//   dx = sigmoid(x) (cos U_c + sin U_s),  dphase = softplus(x) (cos U_s - sin U_c)
// and pass-through dims dx = U.  Key phase derivatives also sum into dbias (per block in LDS,
// then one atomic per dim).  A thread takes 4 consecutive dims per step (D and R are multiples of
// 8; the rows of q, k, dq, dk are 16-byte aligned): 16-byte loads of U, 8-byte loads and stores
// of the bf16 / fp16 rows.
template <typename T>
__device__ __forceinline__ void load4(const uint16_t* p, float* x) {
  const u32x2 w = *reinterpret_cast<const u32x2*>(p);
  x[0] = T::to_float((uint16_t)(w[0] & 0xffffu));
  x[1] = T::to_float((uint16_t)(w[0] >> 16));
  x[2] = T::to_float((uint16_t)(w[1] & 0xffffu));
  x[3] = T::to_float((uint16_t)(w[1] >> 16));
}
template <typename T>
__device__ __forceinline__ void store4(uint16_t* p, const float* g) {
  u32x2 w;
  w[0] = T::pack2(g[0], g[1]);
  w[1] = T::pack2(g[2], g[3]);
  *reinterpret_cast<u32x2*>(p) = w;
}
template <typename T>
__global__ __launch_bounds__(256) void wide_chain_kernel(FlashBwdParams p, const float* wk, const float* wq, int nk) {
  __shared__ float dsum[256];
  const int tid = threadIdx.x;
  const int D = p.D, R = p.R, EP = p.EP;
  if ((int)blockIdx.x < nk) {
    const int nkb = p.NkP / 32;
    const int k0 = 32 * (blockIdx.x % nkb), bhk = blockIdx.x / nkb;
    const int b = bhk / p.Hk, hk = bhk % p.Hk;
    if (k0 >= p.Nk) return;
    for (int d = tid; d < R; d += 256) dsum[d] = 0.f;
    __syncthreads();
    const uint16_t* kb = p.k + (int64_t)b * p.k_s[0] + (int64_t)hk * p.k_s[1];
    uint16_t* dkb = p.dk + (int64_t)b * p.dk_s[0] + (int64_t)hk * p.dk_s[1];
    const float2* tb = R ? p.table + (int64_t)b * p.t_sb + (int64_t)hk * p.t_sh : nullptr;
    float* dfb = p.dfreqs ? p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)hk * p.df_s[1] : nullptr;
    float* kpb = p.kpart ? p.kpart + (int64_t)bhk * p.Nk * R : nullptr;
    const float* wrow = wk + (int64_t)bhk * p.NkP * EP;
    const int D4 = D / 4;
    for (int it = tid; it < 32 * D4; it += 256) {
      const int key = k0 + it / D4, d = 4 * (it % D4);
      if (key >= p.Nk) continue;
      const float* u = wrow + (int64_t)key * EP;
      float g[4];
      if (d < R) {   // R % 4 == 0: all four dims rotated
        float x[4];
        load4<T>(kb + (int64_t)key * p.k_s[2] + d, x);
        const float4 c01 = *reinterpret_cast<const float4*>(tb + (int64_t)key * R + d);
        const float4 c23 = *reinterpret_cast<const float4*>(tb + (int64_t)key * R + d + 2);
        const float4 uc = *reinterpret_cast<const float4*>(u + d), us = *reinterpret_cast<const float4*>(u + R + d);
        const float cs[4] = {c01.x, c01.z, c23.x, c23.z}, sn[4] = {c01.y, c01.w, c23.y, c23.w};
        const float ucv[4] = {uc.x, uc.y, uc.z, uc.w}, usv[4] = {us.x, us.y, us.z, us.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          g[t] = sigmoid_f(x[t]) * (cs[t] * ucv[t] + sn[t] * usv[t]);
          const float dpsi = softplus_f(x[t]) * (cs[t] * usv[t] - sn[t] * ucv[t]);
          if (kpb) {
            kpb[(int64_t)key * R + d + t] = dpsi;
          } else {
            if (dfb) atomicAdd(dfb + (int64_t)key * p.df_s[2] + d + t, dpsi);
            if (p.dbias) atomicAdd(&dsum[d + t], dpsi);
          }
        }
      } else {
        const float4 us = *reinterpret_cast<const float4*>(u + R + d);
        g[0] = us.x; g[1] = us.y; g[2] = us.z; g[3] = us.w;
      }
      store4<T>(dkb + (int64_t)key * p.dk_s[2] + d, g);
    }
    if (p.dbias && !kpb) {
      __syncthreads();
      for (int d = tid; d < R; d += 256) atomicAdd(p.dbias + (int64_t)hk * p.bias_sh + d, dsum[d]);
    }
    return;
  }
  const int nqb = p.NqP / 32, blk = blockIdx.x - nk;
  const int q0 = 32 * (blk % nqb), bh = blk / nqb;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  if (q0 >= p.Nq) return;
  const int q_off = p.Nk - p.Nq;
  const uint16_t* qb = p.q + (int64_t)b * p.q_s[0] + (int64_t)h * p.q_s[1];
  uint16_t* dqb = p.dq + (int64_t)b * p.dq_s[0] + (int64_t)h * p.dq_s[1];
  const float2* tq = R ? p.table + (int64_t)b * p.t_sb + (int64_t)h * p.t_sh : nullptr;
  const float2* bq = R ? p.btab + (p.Hb > 1 ? hk : 0) * R : nullptr;
  float* dfb = p.dfreqs ? p.dfreqs + (int64_t)b * p.df_s[0] + (int64_t)h * p.df_s[1] : nullptr;
  float* qpb = p.qpart && p.dfreqs ? p.qpart + (int64_t)bh * p.Nq * R : nullptr;
  const float* wrow = wq + (int64_t)bh * p.NqP * EP;
  const int D4 = D / 4;
  for (int it = tid; it < 32 * D4; it += 256) {
    const int i = q0 + it / D4, d = 4 * (it % D4);
    if (i >= p.Nq) continue;
    const float* u = wrow + (int64_t)i * EP;
    float g[4];
    if (d < R) {   // R % 4 == 0: all four dims rotated
      float x[4];
      load4<T>(qb + (int64_t)i * p.q_s[2] + d, x);
      const float4 uc = *reinterpret_cast<const float4*>(u + d), us = *reinterpret_cast<const float4*>(u + R + d);
      const float ucv[4] = {uc.x, uc.y, uc.z, uc.w}, usv[4] = {us.x, us.y, us.z, us.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // cos / sin(F[q_off + i] - bias) from the tables of F and of the bias
        const float2 tf = tq[(int64_t)(q_off + i) * R + d + t], tbv = bq[d + t];
        const float cs = fmaf(tf.x, tbv.x, tf.y * tbv.y), sn = fmaf(tf.y, tbv.x, -tf.x * tbv.y);
        g[t] = sigmoid_f(x[t]) * (cs * ucv[t] + sn * usv[t]);
        const float dph = softplus_f(x[t]) * (cs * usv[t] - sn * ucv[t]);
        if (qpb) qpb[(int64_t)i * R + d + t] = dph;
        else if (dfb) atomicAdd(dfb + (int64_t)(q_off + i) * p.df_s[2] + d + t, dph);
      }
    } else {
      const float4 us = *reinterpret_cast<const float4*>(u + R + d);
      g[0] = us.x; g[1] = us.y; g[2] = us.z; g[3] = us.w;
    }
    store4<T>(dqb + (int64_t)i * p.dq_s[2] + d, g);
  }
}

template <typename T, int EP, int DV>
hipError_t fwd_t(const FlashFwdParams& p, hipStream_t s) {
  return launch_named("flash_wide_fwd", wide_fwd_kernel<T, EP, DV>, dim3((p.NqP / 128) * p.B * p.Hq), dim3(256), s, p);
}

// Column chunks per row block (each chunk recomputes the scores), as few as measured fastest: with
// the tiles loaded straight into LDS, one dK/dV chunk at 256 features and two at 384 / 512, one
// dQ chunk at 256 and two at 384 / 512 (some of these spill a few registers, which still beats
// recomputing the scores more often).
template <int EP>
constexpr int kv_chunks() { return EP <= 256 ? 1 : 2; }
template <int EP>
constexpr int q_chunks() { return EP <= 256 ? 1 : 2; }

template <typename T, int EP, int DV>
hipError_t bwd_t(const FlashBwdParams& p, float* wk, float* wq, hipStream_t s) {
  constexpr int CK = kv_chunks<EP>(), CQ = q_chunks<EP>();
  hipError_t e = launch_named("flash_wide_kv", wide_kv_kernel<T, EP, DV, CK>, dim3((p.NkP / (128 / CK)) * p.B * p.Hk),
                              dim3(256), s, p, wk);
  if (e != hipSuccess) return e;
  e = launch_named("flash_wide_q", wide_q_kernel<T, EP, DV, CQ>, dim3((p.NqP / (128 / CQ)) * p.B * p.Hq), dim3(256), s,
                   p, wq);
  if (e != hipSuccess) return e;
  const int nk = (p.NkP / 32) * p.B * p.Hk, nq = (p.NqP / 32) * p.B * p.Hq;
  return launch_named("flash_wide_chain", wide_chain_kernel<T>, dim3(nk + nq), dim3(256), s, p,
                      (const float*)wk, (const float*)wq, nk);
}

}  // namespace

bool flash_wide_shape(int EP, int DV) { return DV == 256 && (EP == 256 || EP == 384 || EP == 512); }

hipError_t launch_flash_wide_fwd(const FlashFwdParams& p, int dtype, hipStream_t s) {
  if (!flash_wide_shape(p.EP, p.DV)) return hipErrorInvalidValue;
  if (dtype == 2) {
    if (p.EP == 256) return fwd_t<BF16, 256, 256>(p, s);
    if (p.EP == 384) return fwd_t<BF16, 384, 256>(p, s);
    return fwd_t<BF16, 512, 256>(p, s);
  }
  if (p.EP == 256) return fwd_t<F16, 256, 256>(p, s);
  if (p.EP == 384) return fwd_t<F16, 384, 256>(p, s);
  return fwd_t<F16, 512, 256>(p, s);
}

hipError_t launch_flash_wide_bwd(const FlashBwdParams& p, float* wk, float* wq, int dtype, hipStream_t s) {
  if (!flash_wide_shape(p.EP, p.DV)) return hipErrorInvalidValue;
  if (dtype == 2) {
    if (p.EP == 256) return bwd_t<BF16, 256, 256>(p, wk, wq, s);
    if (p.EP == 384) return bwd_t<BF16, 384, 256>(p, wk, wq, s);
    return bwd_t<BF16, 512, 256>(p, wk, wq, s);
  }
  if (p.EP == 256) return bwd_t<F16, 256, 256>(p, wk, wq, s);
  if (p.EP == 384) return bwd_t<F16, 384, 256>(p, wk, wq, s);
  return bwd_t<F16, 512, 256>(p, wk, wq, s);
}

}  // namespace pope
