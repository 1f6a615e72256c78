// Flash attention forward with PoPE fused in (bf16 / fp16 MFMA, gfx950).
//
// Reference semantics: triton_pope_flash_attn.py:23-117 (kernel) and :222-271
// (launcher); PyTorch path attention.py:106-145.
//
// Inputs come from the shared preparation (flash_prep.hip): K_hat rows, Q_hat rows pre-scaled
// by softmax_scale * log2(e) (so S = Q_hat K_hat^T is the score in log2 units) and the key
// visibility words.  V is read from the caller's tensor.
//
// Work decomposition
//   one workgroup = 8 waves = 128 query rows of one (batch, query head).  Waves 0-3 (group 0)
//   and 4-7 (group 1) own the same 128 rows, 32 per wave, and split the key axis: the
//   workgroup stages pairs of BN-key tiles, group g takes tile 2 t + g.  Each group keeps its
//   own online-softmax state; group 1 hands (m, l, O) to group 0 through LDS at the end.
// Staging
//   K_hat and V tiles go straight from global memory into LDS (global_load_lds_dwordx4, no
//   registers), into a ring of stage slots: while pair t is consumed, pair t + 1 is resident
//   and pair t + 2 (four slots, where they fit the LDS: also pair t + 3) is in flight.  Tiles
//   are unpadded and XOR-swizzled (tile_swz).
// Per wave and tile
//   S^T = K_hat Q_hat^T on v_mfma_f32_32x32x16: A = K_hat rows from LDS (lane = key), B = the
//   wave's Q_hat rows held in registers (lane = query), so every query's scores sit in one
//   lane pair and the softmax reductions stay in-lane (plus one permlane32 swap).  The
//   accumulator starts from -m (the running reference max), so the MFMA returns s - m.
//   O^T += V^T P^T takes the probabilities straight from the S registers as the B operand; V^T
//   comes from the row-major V tile through LDS transpose reads in the same key order.
//   The scores of tile t + 1 are multiplied while the softmax of tile t runs on the VALU.
// Online softmax
//   p = exp2(s - m) with a lazily updated reference m: m moves only when a row's tile maximum
//   exceeds it by more than 8 (p <= 2^8 stays exact in fp32 / bf16 range), or on the row's
//   first visible key.  The row sum is taken from the bf16 probabilities that feed the MFMA
//   (v_dot2_f32_bf16 against (1, 1)).
// Masking
//   top-left causal (key j visible to query i iff j <= i, the SDPA convention the reference
//   uses, triton_pope_flash_attn.py:64,86-87), key padding mask (nonzero = keep), keys >= Nk.
//   Tiles past the causal diagonal or past the batch's last visible key are never loaded.
//   Fully masked rows give O = 0 and LSE = -inf (:114,117).
// Scheduling
//   blockIdx -> (query block, batch*head) with the heaviest causal blocks first and
//   batch*head fastest, so every workgroup of one (batch, head) lands on the same XCD (the
//   dispatcher deals workgroup ids round-robin over the 8 XCDs) and its K_hat / V stay in one
//   L2.  One workgroup per CU; twice as many workgroups as CUs balance the causal triangle.
#include "pope_common.hpp"
#include "pope_kernels.hpp"

namespace pope {

namespace {

constexpr int kBM = 128;        // query rows per workgroup
constexpr int kThreads = 512;   // 8 waves

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

template <int EP, int DV>
struct FwdCfg {
  static constexpr int BN = (EP + DV <= 192 && DV <= 64) ? 64 : 32;   // keys per tile
  static constexpr int KB = BN / 32;                                  // 32-key blocks per tile
  static constexpr int KS = EP / 16;                                  // 16-wide k steps of S
  static constexpr int NDB = DV / 32;                                 // 32-row blocks of O^T
  static constexpr int EPU = EP / 8, DVU = DV / 8;                    // 16-byte units per row
  static constexpr int KTILE = BN * EP;                               // elements per K_hat tile
  static constexpr int VTILE = BN * DV;
  static constexpr int STAGE = 2 * (KTILE + VTILE) * 2;               // bytes per stage slot
  static constexpr int UNITS = STAGE / 16;
  static constexpr int KUNITS = 2 * KTILE / 8;
  static constexpr int LPT = (UNITS + kThreads - 1) / kThreads;       // direct loads per thread
  // loads per pair of the last wave (the fewest: the last load of a pair can be partial)
  static constexpr int LMIN = (UNITS - (kThreads - 64) + kThreads - 1) / kThreads;
  // stage slots: pair t's V and pair t + 1's K_hat in use, SLOTS - 2 pairs loading ahead (four
  // where they fit the LDS, except for 128-wide V rows, whose registers the deeper ring spills)
  static constexpr int SLOTS = 4 * STAGE <= 160 * 1024 && DV < 128 ? 4 : 3;
  static constexpr int MS = 3 + 16 * NDB;                             // floats per lane in the merge
  static constexpr int MERGE = 4 * 64 * MS * 4;
  static constexpr int LDS = SLOTS * STAGE > MERGE ? SLOTS * STAGE : MERGE;
  static_assert(KUNITS % 64 == 0 && UNITS % 64 == 0, "loads must split at wave boundaries");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <typename T, int EP, int DV>
__global__ __launch_bounds__(kThreads, 1) void flash_fwd_kernel(FlashFwdParams p) {
  typedef FwdCfg<EP, DV> C;
  constexpr int BN = C::BN, KB = C::KB, KS = C::KS, NDB = C::NDB;
  typedef typename T::vec8 vec8;

  __shared__ __attribute__((aligned(16))) char smem[C::LDS];

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lr = lane & 31, hf = lane >> 5;
  const int grp = wave >> 2, wq = wave & 3;
  const int BH = p.B * p.Hq;
  const int bh = blockIdx.x % BH;
  const int qb = p.nqb - 1 - (int)(blockIdx.x / BH);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h % p.Hk;
  const int Nk = p.Nk, Nq = p.Nq, D = p.D;
  const int qw0 = qb * kBM + wq * 32;   // first query row of this wave
  const int qi = qw0 + lr;

  // ---- the wave's Q_hat rows as MFMA B operands --------------------------------
  vec8 qreg[KS];
  {
    const uint16_t* qrow = p.qh + ((int64_t)bh * p.NqP + qi) * EP;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qreg[kk] = as_vec8<vec8>(ld16(qrow + 16 * kk + 8 * hf));
  }
  settle_vector_loads();

  // ---- key range: causal bound of the block's last query, last visible key of the batch ----
  // (the preparation's words and bounds are read-only here: the constant address space lets
  // the uniform reads go through scalar loads)
  typedef const __attribute__((address_space(4))) uint64_t cu64;
  typedef const __attribute__((address_space(4))) int ci32;
  int nkeys = min(((ci32*)p.kend)[b], Nk);
  if (p.causal) nkeys = min(nkeys, min(qb * kBM + kBM, Nq));
  const int nt = (nkeys + BN - 1) / BN;
  const int npair = (nt + 1) / 2;
  cu64* mw = (cu64*)p.mwords + (int64_t)b * p.NW;

  // ---- direct-load plan: unit c = m * 512 + tid of a stage slot ---------------------
  // K_hat units first (tile g, row r, swizzled unit), then V units.  Offsets are relative
  // to the pair's first key row j0.
  const uint16_t* khg = p.kh + (int64_t)(b * p.Hk + hk) * p.NkP * EP;
  const uint16_t* vg = p.v + (int64_t)b * p.v_s[0] + (int64_t)hk * p.v_s[1];
  const int vs2 = (int)p.v_s[2];
  // one offset per load: K_hat element offset relative to the pair's first row; V element
  // offset of (row, column) relative to the pair's first row (rows past Nk clamp to the last
  // chunk of the last row: their P is 0; columns past D repeat the last chunk and are never stored)
  int ld_o[C::LPT];
#pragma unroll
  for (int m = 0; m < C::LPT; ++m) {
    const int c = m * kThreads + tid;
    if (c < C::KUNITS) {
      const int g = c / (BN * C::EPU), rem = c % (BN * C::EPU);
      const int r = rem / C::EPU, u = (rem % C::EPU) ^ tile_swz(C::EPU, r);
      ld_o[m] = (g * BN + r) * EP + 8 * u;
    } else {
      const int cv = c - C::KUNITS;
      const int g = cv / (BN * C::DVU), rem = cv % (BN * C::DVU);
      const int r = rem / C::DVU, u = (rem % C::DVU) ^ tile_swz(C::DVU, r);
      ld_o[m] = (g * BN + r) * vs2 + min(8 * u, D - 8);
    }
  }
  const int v_last = (Nk - 1) * vs2 + D - 8;   // start of the last chunk of the last row
  auto issue = [&](int pr) {
    char* slot = smem + (pr % C::SLOTS) * C::STAGE;
    const int j0 = pr * 2 * BN;
    const uint16_t* kp = khg + j0 * EP;   // K_hat rows are padded to NkP: no clamp
    const int vrow0 = j0 * vs2;
#pragma unroll
    for (int m = 0; m < C::LPT; ++m) {
      const int c0 = m * kThreads + wave * 64;   // first unit of this wave's instruction
      const uint32_t dst = lds_addr(slot + c0 * 16);
      const uint16_t* vsrc = vg + min(vrow0 + ld_o[m], v_last);
      if ((m + 1) * kThreads <= C::KUNITS) {          // K_hat units for every wave
        load_lds16(kp + ld_o[m], dst);
      } else if (m * kThreads >= C::KUNITS) {         // V units
        if (C::UNITS % kThreads == 0 || c0 < C::UNITS) load_lds16(vsrc, dst);
      } else {                                        // the K / V boundary falls in this load
        load_lds16(c0 < C::KUNITS ? (const void*)(kp + ld_o[m]) : (const void*)vsrc, dst);
      }
    }
  };

  // K_hat A operand: row 32 kb + lr, unit 2 kk + hf of tile grp; V^T A operand: transpose reads
  const TileOffsets<C::EPU> ko(lane);
  const TileOffsets<C::DVU> vo(lane);

  // ---- state -----------------------------------------------------------------------------
  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  f32x16 negm;   // -m in every register: the initial accumulator of S
#pragma unroll
  for (int r = 0; r < 16; ++r) negm[r] = 0.f;
  float m_ref = 0.f, l_run = 0.f;
  bool m_set = false;
  f32x16 sacc[KB];
  auto kh_tile = [&](int pr) -> const uint16_t* {
    return reinterpret_cast<const uint16_t*>(smem + (pr % C::SLOTS) * C::STAGE) + grp * C::KTILE;
  };
  auto v_tile = [&](int pr) -> const uint16_t* {
    return reinterpret_cast<const uint16_t*>(smem + (pr % C::SLOTS) * C::STAGE) + 2 * C::KTILE + grp * C::VTILE;
  };
  // Visibility of the group's tile of pair pr: true when every key is visible to every row of
  // the wave (no per-element mask needed).
  auto tile_full = [&](int pr, uint64_t& mb) -> bool {
    const int tile = 2 * pr + grp;
    const int j0 = tile * BN;
    mb = 0;
    if (tile < nt) {
      mb = mw[j0 >> 6];
      if (BN == 32) mb = (mb >> (j0 & 32)) & 0xffffffffull;
    }
    const uint64_t all = BN == 64 ? ~0ull : 0xffffffffull;
    return mb == all && !(p.causal && j0 + BN - 1 > qw0);
  };
  // masked scores -> -inf (cold: diagonal and partially visible tiles)
  auto apply_mask = [&](int pr, uint64_t mb, f32x16* s) {
    const int j0 = (2 * pr + grp) * BN;
    // the lane's keys are 32 kb + 8 (r >> 2) + (r & 3) past 4 hf: compile-time bit positions
    const uint64_t w = mb >> (4 * hf);
    const int lim = p.causal ? qi - j0 - 4 * hf : BN;   // causal: key offset <= lim
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 32 * kb + 8 * (r >> 2) + (r & 3);
        const bool ok = ((uint32_t)(w >> kr) & 1u) && kr <= lim;
        // in place (tied operand), so the scores keep their registers across the branch
        asm("v_cmp_ne_u32 vcc, 0, %2\n\tv_cndmask_b32 %0, %1, %0, vcc"
            : "+v"(s[kb][r]) : "v"(-INFINITY), "v"((int)ok) : "vcc");
      }
  };
  // S^T - m for the group's tile of pair pr (the accumulators start from the -m block).
  constexpr int NQK = KB * KS;
  // Rows of up to 128 expanded features run the step's two bursts in the fenced order below,
  // with six K_hat operand reads in flight, so that an operand read's LDS latency overlaps the
  // products before it instead of preceding each product (C3 forward 55.0 -> 53.5 us).  Wider
  // rows keep the compiler's interleave (sched_group_barrier), which was faster there (C4 86.9
  // against 88.5 us).
  constexpr bool kFenced = EP <= 128;
  constexpr int kPF = 6;   // K_hat operand reads in flight ahead of the products (fenced order)
  auto k_operand = [&](const uint16_t* kt, int i) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(kt + 32 * (i / KS) * EP + ko.row_at(i % KS));
  };
  auto qk = [&](int pr, f32x16* s) {
    const uint16_t* kt = kh_tile(pr);
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      const int kb = i / KS, kk = i % KS;
      s[kb] = T::mfma32(as_vec8<vec8>(k_operand(kt, i)), qreg[kk], kk == 0 ? negm : s[kb]);
    }
  };
  auto rowmax = [&](const f32x16* s) -> float {
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    return half_swap_max(mt);
  };
  // lazy reference update (rare, wave-uniform branch): moves m when a row's tile maximum mt
  // (relative to m) exceeds 8, or on the row's first visible key
  auto rescale = [&](float mt, f32x16* s) {
    const bool need = (mt > -INFINITY) & (!m_set | (mt > 8.f));
    if (__any(need)) {
      POPE_COLD_PATH();
      const float sh = need ? mt : 0.f;
      const float alpha = (need && m_set) ? __builtin_amdgcn_exp2f(-mt) : 1.f;
      // in-place updates (tied operands): the values keep their registers across the branch
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) asm("v_mul_f32 %0, %0, %1" : "+v"(oacc[db][r]) : "v"(alpha));
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) asm("v_sub_f32 %0, %0, %1" : "+v"(s[kb][r]) : "v"(sh));
      asm("v_mul_f32 %0, %0, %1" : "+v"(l_run) : "v"(alpha));
      m_ref += sh;
      m_set = m_set || need;
#pragma unroll
      for (int r = 0; r < 16; ++r) asm("v_mov_b32 %0, %1" : "=v"(negm[r]) : "v"(-m_ref));
    }
  };
  // probabilities (bf16 / fp16 pairs, in B-operand order) and the row sum
  auto probs = [&](const f32x16* s, u32x4* pw) {
    const uint32_t ones = T::pack2(1.f, 1.f);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t w = T::pack2(__builtin_amdgcn_exp2f(s[kb][8 * g + 2 * q]),
                                      __builtin_amdgcn_exp2f(s[kb][8 * g + 2 * q + 1]));
          pw[2 * kb + g][q] = w;
          l_run = T::dot2(w, ones, l_run);
        }
  };
  // The pipelined step's two product bursts, each in an explicit order: a fence
  // (sched_barrier) after every product pins, next to that product, the operand reads of a later
  // product (so an LDS read has several products' time to land, instead of preceding each
  // product) and an even share of the VALU work the burst overlaps.
  //   scores of tile t + 1  with  the probabilities and row sum of tile t
  //   P V of tile t          with  the row maximum of tile t + 1
  constexpr int NPU = 2 * KB * 4;   // probability units: 2 exponentials, a pack, a row-sum dot
  auto prob_unit = [&](const f32x16* s, u32x4* pw, int u) {
    const int kb = u / 8, g = (u / 4) % 2, q = u % 4;
    const uint32_t w = T::pack2(__builtin_amdgcn_exp2f(s[kb][8 * g + 2 * q]),
                                __builtin_amdgcn_exp2f(s[kb][8 * g + 2 * q + 1]));
    pw[2 * kb + g][q] = w;
    l_run = T::dot2(w, T::pack2(1.f, 1.f), l_run);
    // pinned here (a volatile statement stays between the fences around it): otherwise the
    // packs and the row sum drift past the fences into a later block
    asm volatile("" : "+v"(pw[2 * kb + g][q]), "+v"(l_run));
  };
  auto qk_probs = [&](int pr, f32x16* s, const f32x16* cur, u32x4* pw) {
    const uint16_t* kt = kh_tile(pr);
    u32x4 fk[NQK];
#pragma unroll
    for (int i = 0; i < kPF && i < NQK; ++i) fk[i] = k_operand(kt, i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      const int kb = i / KS, kk = i % KS;
      s[kb] = T::mfma32(as_vec8<vec8>(fk[i]), qreg[kk], kk == 0 ? negm : s[kb]);
      if (i + kPF < NQK) fk[i + kPF] = k_operand(kt, i + kPF);
#pragma unroll
      for (int u = i * NPU / NQK; u < (i + 1) * NPU / NQK; ++u) prob_unit(cur, pw, u);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  constexpr int NPV = (BN / 16) * NDB, kVPF = 2;
  auto pv_rowmax = [&](int pr, const u32x4* pw, const f32x16* s) -> float {
    const uint32_t vb = lds_addr(v_tile(pr));
    uint32_t alo[NDB], ahi[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      alo[db] = opaque_u32(vb + 2 * vo.lo_at(db));
      ahi[db] = opaque_u32(vb + 2 * vo.hi_at(db));
    }
    auto v_operand = [&](int i) -> u32x4 {
      const int g16 = i / NDB, db = i % NDB;
      const uint32_t off = 2 * 16 * g16 * DV;
      return lds_tr8_at(alo[db] + off, ahi[db] + off);
    };
    u32x4 fv[NPV];
#pragma unroll
    for (int i = 0; i < kVPF && i < NPV; ++i) fv[i] = v_operand(i);
    __builtin_amdgcn_sched_barrier(0);
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
      const int g16 = i / NDB, db = i % NDB;
      oacc[db] = T::mfma32(as_vec8<vec8>(fv[i]), as_vec8<vec8>(pw[g16]), oacc[db]);
      if (i + kVPF < NPV) fv[i + kVPF] = v_operand(i + kVPF);
#pragma unroll
      for (int x = i * 16 * KB / NPV; x < (i + 1) * 16 * KB / NPV; ++x) mt = fmaxf(mt, s[x / 16][x % 16]);
      asm volatile("" : "+v"(mt));
      __builtin_amdgcn_sched_barrier(0);
    }
    return half_swap_max(mt);
  };
  // O^T += V^T P^T over the tile's 16-key groups
  auto pv = [&](int pr, const u32x4* pw) {
    // one address register per (db, row run); the 16-key groups are immediate offsets
    const uint32_t vb = lds_addr(v_tile(pr));
    uint32_t alo[NDB], ahi[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      alo[db] = opaque_u32(vb + 2 * vo.lo_at(db));
      ahi[db] = opaque_u32(vb + 2 * vo.hi_at(db));
    }
#pragma unroll
    for (int g16 = 0; g16 < BN / 16; ++g16) {
      const vec8 pb = as_vec8<vec8>(pw[g16]);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint32_t off = 2 * 16 * g16 * DV;
        oacc[db] = T::mfma32(as_vec8<vec8>(lds_tr8_at(alo[db] + off, ahi[db] + off)), pb, oacc[db]);
      }
    }
  };

  // ---- main loop ---------------------------------------------------------------------
  // Iteration t: reference update for tile t; masks of tile t + 1 folded into its initial
  // accumulators; then the score MFMAs of tile t + 1 interleaved with the exponentials of
  // tile t, and the P V MFMAs of tile t interleaved with the row maximum of tile t + 1.
  if (npair > 0) {
    // pairs 0 .. SLOTS - 2 in flight; wait for pair 0 (every wave issues at least LMIN loads per
    // pair, so allowing that many per later pair never lets one of pair 0's through)
    issue(0);
    if (npair > 1) issue(1);
    if (C::SLOTS > 3 && npair > 2) issue(2);
    if (C::SLOTS > 3 && npair > 2) wait_vmcnt<2 * C::LMIN>();
    else if (npair > 1) wait_vmcnt<C::LMIN>();
    else wait_vmcnt<0>();
    __syncthreads();
    uint64_t mb0;
    const bool full0 = tile_full(0, mb0);
    qk(0, sacc);
    if (!full0) {
      POPE_COLD_PATH();
      apply_mask(0, mb0, sacc);
    }
    float mt = rowmax(sacc);
    // one pipelined step: tile t in `cur` (scores - m), tile t + 1 computed into `nxt`
    auto step = [&](int t, f32x16* cur, f32x16* nxt) {
      rescale(mt, cur);
      u32x4 pw[2 * KB];
      uint64_t mb;
      const bool full = tile_full(t + 1, mb);
      // this thread's loads of pair t + 1 landed (with four slots pair t + 2 may be in flight)
      if (C::SLOTS > 3 && t + 2 < npair) wait_vmcnt<C::LMIN>();
      else wait_vmcnt<0>();
      __syncthreads();      // ... everyone's; and pair t - 1's slot is free
      if (t + C::SLOTS - 1 < npair) issue(t + C::SLOTS - 1);
      // keep the exponentials of tile t below the barrier, next to the MFMAs they overlap
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) asm volatile("" : "+v"(cur[kb]));
      if constexpr (kFenced) {
        qk_probs(t + 1, nxt, cur, pw);
      } else {
        qk(t + 1, nxt);
        probs(cur, pw);
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedValu, (6 * KB * 16 / 2) / NQK, 0);
        }
      }
      // the packed probabilities are complete here, before the mask branch: otherwise their
      // exponentials sink past it into the P V block, away from the score products they overlap
#pragma unroll
      for (int i = 0; i < 2 * KB; ++i) asm volatile("" : "+v"(pw[i]));
      if (!full) {
        POPE_COLD_PATH();
        apply_mask(t + 1, mb, nxt);
      }
      if constexpr (kFenced) {
        mt = pv_rowmax(t, pw, nxt);
      } else {
        pv(t, pw);
        mt = rowmax(nxt);
#pragma unroll
        for (int i = 0; i < NPV; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 1);
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 1);
          __builtin_amdgcn_sched_group_barrier(kSchedValu, 2, 1);
        }
      }
    };
    auto last = [&](int t, f32x16* cur) {
      rescale(mt, cur);
      u32x4 pw[2 * KB];
      probs(cur, pw);
      pv(t, pw);
    };
    // unrolled by two so the score buffers alternate instead of being copied
    f32x16 sb[KB];
    int t = 0;
    for (; t + 2 < npair; t += 2) {
      step(t, sacc, sb);
      step(t + 1, sb, sacc);
    }
    if (t + 1 < npair) {
      step(t, sacc, sb);
      last(t + 1, sb);
    } else {
      last(t, sacc);
    }
  }

  // ---- merge group 1 into group 0, epilogue ------------------------------------------
  __syncthreads();   // every wave is done with the stage slots
  float* mg = reinterpret_cast<float*>(smem);
  const float m_eff = m_set ? m_ref : -INFINITY;
  if (grp == 1) {
    float* dst = mg + (wq * 64 + lane) * C::MS;
    dst[0] = m_eff;
    dst[1] = l_run;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[2 + 16 * db + r] = oacc[db][r];
  }
  __syncthreads();
  if (grp == 1) return;
  float m_fin;
  {
    const float* src = mg + (wq * 64 + lane) * C::MS;
    const float m1 = src[0], l1 = src[1];
    const float m_new = fmaxf(m_eff, m1);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float a0 = __builtin_amdgcn_exp2f(m_eff - m_use), a1 = __builtin_amdgcn_exp2f(m1 - m_use);
    l_run = l_run * a0 + l1 * a1;
    m_fin = m_new;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] = oacc[db][r] * a0 + src[2 + 16 * db + r] * a1;
  }
  const float l = l_run + wave_shfl_xor(l_run, 32);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (qi < Nq) {
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
          m_fin == -INFINITY ? -INFINITY : (m_fin + __builtin_amdgcn_logf(l)) * kLn2;
  }
}

template <typename T, int EP, int DV>
hipError_t launch_t(const FlashFwdParams& p, hipStream_t s) {
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

}  // namespace pope
