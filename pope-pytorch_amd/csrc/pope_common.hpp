// Shared device helpers for the PoPE kernels (gfx950 / CDNA4, wave64).
//
// The polar transform of PoPE (reference pope.py:30-86, triton_pope.py:18-24):
//   magnitude  a = softplus(x)            (beta = 1, threshold 20: x > 20 -> x)
//   phase      query: phi = F[q_off + i, d]      key: psi = F[j, d] + bias[h, d]
//   expanded   x_hat = [a cos(phase) | a sin(phase) | raw pass-through dims]
// Every kernel lays the expanded feature axis out as E = D + R columns:
//   e <  R        -> cos part of rotated dim e
//   R <= e < 2R   -> sin part of rotated dim e - R
//   e >= 2R       -> pass-through dim e - R (raw, no softplus)
// The column order inside a kernel is free (it only changes the order of a
// dot product); the public materialising transform interleaves (pope.py:70).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pope {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element-type traits for the half-precision MFMA paths.
struct BF16 {
  static constexpr int kCode = 2;   // pope_dtype code
  typedef __bf16 scalar;
  typedef bf16x8 vec8;
  static __device__ __forceinline__ float to_float(uint16_t bits) {
    return __uint_as_float(((uint32_t)bits) << 16);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ uint16_t bits(float a) { return __builtin_bit_cast(uint16_t, (__bf16)a); }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // c + a.x * b.x + a.y * b.y on packed pairs (v_dot2_f32_bf16)
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  }
};

struct F16 {
  static constexpr int kCode = 1;
  typedef _Float16 scalar;
  typedef f16x8 vec8;
  static __device__ __forceinline__ float to_float(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ uint16_t bits(float a) { return __builtin_bit_cast(uint16_t, (_Float16)a); }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  // c + a.x * b.x + a.y * b.y on packed pairs (v_dot2_f32_f16)
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  }
};

// softplus in fp32 with hardware exp2/log2: max(x, 0) + ln(1 + e^-|x|).  For |x| > 16.6,
// e^-|x| < 2^-24 and fl(1 + e^-|x|) = 1, so the result is max(x, 0) exactly: the
// reference's threshold (x > 20 -> x, beta = 1) holds without a test.
__device__ __forceinline__ float softplus_f(float x) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e);
  return fmaf(__builtin_amdgcn_logf(1.f + e), kLn2, fmaxf(x, 0.f));
}

// d softplus / dx = sigmoid(x).
__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// Accurate fp32 sine/cosine with full range reduction (device math library).
__device__ __forceinline__ void sincos_acc(float x, float* s, float* c) { sincosf(x, s, c); }

// sin / cos of x (radians): x / 2pi as an FMA-split product (about 2^-40 absolute for |x| < 2^24),
// its fraction, and the hardware sine / cosine of revolutions (v_sin_f32 / v_cos_f32).  Measured
// maximum absolute error 2e-7 for |x| up to 1e6.
__device__ __forceinline__ void sincos_rev(float x, float* s, float* c) {
#pragma clang fp contract(off)   // hi must stay the rounded product: contracted, lo would count twice
  constexpr float kHi = 0.15915494f;                                          // fl(1 / 2pi)
  constexpr float kLo = (float)(0.15915494309189533577 - (double)0.15915494f);   // 1 / 2pi - kHi
  const float hi = x * kHi;
  const float lo = fmaf(x, kHi, -hi) + x * kLo;
  const float fr = (hi - __builtin_rintf(hi)) + lo;   // hi - rint(hi) is exact
  *s = __builtin_amdgcn_sinf(fr);
  *c = __builtin_amdgcn_cosf(fr);
}


__device__ __forceinline__ uint32_t u16lo(uint32_t w) { return w & 0xffffu; }
__device__ __forceinline__ uint32_t u16hi(uint32_t w) { return w >> 16; }

template <typename V>
__device__ __forceinline__ V as_vec8(u32x4 w) { return __builtin_bit_cast(V, w); }

// 8 consecutive 16-bit elements -> 8 floats.
template <typename T>
__device__ __forceinline__ void unpack8(u32x4 w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = T::to_float((uint16_t)u16lo(w[i]));
    f[2 * i + 1] = T::to_float((uint16_t)u16hi(w[i]));
  }
}

// XCD-aware workgroup remap. Consecutive hardware workgroup ids are dealt
// round-robin to the 8 XCDs of an MI355X; each XCD has its own L2.  Return a
// logical id such that each XCD processes a contiguous range of logical ids
// (so the K/V of one (batch, head) stays in one L2).
__device__ __forceinline__ int xcd_remap(int hw_id, int total) {
  constexpr int kXcd = 8;
  if (total % kXcd != 0) return hw_id;
  int per = total / kXcd;
  return (hw_id % kXcd) * per + hw_id / kXcd;
}

__device__ __forceinline__ float wave_shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// max(v[lane], v[lane ^ 32]) with one v_permlane32_swap: swapping the upper half of a copy of v
// with the lower half of another leaves lane l holding v[l] and v[l ^ 32] in the two outputs.
__device__ __forceinline__ float half_swap_max(float v) {
  const int x = __builtin_bit_cast(int, v);
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}

// Marks a rarely taken branch body so the compiler keeps it a branch instead of
// speculating it into per-lane selects on every path.
#define POPE_COLD_PATH() asm volatile("")

// Wave index within the workgroup as a scalar: the compiler's divergence analysis then
// treats conditions on it as uniform and emits scalar branches instead of per-lane selects.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// LDS row strides.  The LDS serves 64 banks of 4 bytes; counted in 16-byte
// units, a 128-bit row read by 16 lanes (rows r0..r0+15, one unit each) is
// conflict-free when the row stride is odd, and a transpose read by 32 lanes
// (4 rows x 4 consecutive units, lds_operand_tr) when the stride is 4 or 12
// mod 16.  A tile read both ways takes a stride of 4 or 12 mod 16 units and
// swizzles: unit u of row r lives at u ^ ((r >> 2) & 3) (rows of one transpose
// read share the swizzle; 16 consecutive rows spread over all 16 bank groups).
__host__ __device__ constexpr int lds_units_rows(int units) { return units | 1; }
__host__ __device__ constexpr int lds_units_tr(int units) {
  return (units % 16 == 4 || units % 16 == 12) ? units : lds_units_tr(units + 4 - units % 4);
}
__device__ __forceinline__ int lds_swz(int row, int unit) { return unit ^ ((row >> 2) & 3); }

// XOR swizzle of the 16-byte units of an unpadded LDS tile whose rows hold U units (U a
// multiple of 4): unit u of row r is stored at r * U + (u ^ tile_swz(U, r)).  The value depends
// on r % 16 only and keeps u within its row.  With it, both reads the MFMA operands make are
// free of bank conflicts (64 banks of 4 bytes = 16 units):
//   row read        16 lanes read unit u of 16 consecutive rows (ds_read_b128);
//   transpose read  4 consecutive rows (aligned to 4) x 4 consecutive units (aligned to 4)
//                   (ds_read_b64_tr_b16, lds_read_tr16).
// Unpadded rows let tiles be filled by direct global-to-LDS loads, which write 64 consecutive
// units per wave instruction.
__host__ __device__ constexpr int tile_swz(int U, int r) {
  return (U % 16 == 0) ? (((r & 3) << 2) | ((r >> 2) & 3))
         : (U % 8 == 0) ? ((((r >> 1) & 1) << 2) | ((r >> 2) & 3))
                        : ((r >> 2) & 3);
}

// LDS transpose read (ds_read_b64_tr_b16).  Within each group of 16 lanes, lane
// j supplies the address of 4 consecutive 16-bit elements; output lane 4a + c
// receives element c of the chunks addressed by lanes a, a + 4, a + 8, a + 12
// (in that order).  Pointed at rows r0 + j / 4 and columns n0 + 4 (j % 4) of a
// row-major tile, every lane gets 4 consecutive rows of its own column n0 + j.
typedef __attribute__((ext_vector_type(4))) short v4i16;
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16 __attribute__((address_space(3)))*)p);
  return __builtin_bit_cast(u32x2, r);
}

// The same read at an LDS byte address.  With `a` made opaque (opaque_u32) once per tile, the
// constant part of every read's address folds into the instruction's offset field instead of
// costing an address register and one or two VALU instructions per read.
__device__ __forceinline__ u32x2 lds_read_tr16_at(uint32_t a) {
  typedef v4i16 __attribute__((address_space(3))) * lds_v4i16_ptr;
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(size_t)a);
  return __builtin_bit_cast(u32x2, r);
}
__device__ __forceinline__ u32x4 lds_tr8_at(uint32_t lo, uint32_t hi) {
  const u32x2 a = lds_read_tr16_at(lo);
  const u32x2 b = lds_read_tr16_at(hi);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// A value the compiler may not re-derive or re-associate (it stays the one register it is).
__device__ __forceinline__ uint32_t opaque_u32(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Direct global -> LDS load of 16 bytes per lane: lane l's bytes land at LDS byte address
// lds + 16 l (lds is wave-uniform, passed in M0).  Written as inline assembly so that the
// compiler does not add its conservative wait for every outstanding LDS load before each LDS
// read: the kernel waits for its own loads (vmcnt) before the barrier that publishes a stage.
__device__ __forceinline__ void load_lds16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory");
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Waits until at most n of this thread's vector memory loads are outstanding.
#define POPE_WAIT_VMCNT(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")

// The same with the count as a template argument.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits for every outstanding vector memory load, as an instruction the compiler's own wait
// insertion accounts for: registers loaded before it count as ready afterwards, so no later
// use of them (inside a loop that also has direct-to-LDS loads in flight) adds a vmcnt(0).
__device__ __forceinline__ void settle_vector_loads() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// Instruction-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedValu = 0x002, kSchedMfma = 0x008, kSchedDsRead = 0x100;

// Number of distinct low-bit patterns tile_swz can flip: swizzle values stay below 4 (U % 16 in
// {4, 12}), 8 (U % 16 == 8) or 16 (U % 16 == 0).
__host__ __device__ constexpr int swz_bits(int U) { return U % 16 == 0 ? 4 : U % 8 == 0 ? 3 : 2; }

// Operand offsets (elements) of the MFMA reads of a row-major tile of U 16-byte units per row
// stored with tile_swz.  The swizzle only flips the low swz_bits(U) bits of a unit index, so
// the lane-dependent part repeats with a short period and a few base registers serve every
// k step / column block:
//   row read   lane % 32 reads row lane % 32, unit 2 kk + lane / 32        (ds_read_b128)
//   transpose  rows R0 + 4 h + j / 4 and R0 + 8 + 4 h + j / 4, columns 32 nb + 8 u + 4 (j & 1),
//              j = lane % 16, h = lane / 32, u = 2 (lane / 16 % 2) + (j / 2 % 2)
//              (two lds_read_tr16 chunks; the k order is the register order of a 32x32 MFMA
//              result read back as an operand: [4 h, 4 h + 4) then [8 + 4 h, 12 + 4 h))
template <int U>
struct TileOffsets {
  static constexpr int RP = 1 << (swz_bits(U) - 1);   // period of the row-read offset in kk
  static constexpr int TP = 1 << (swz_bits(U) - 2);   // period of the transpose offset in nb
  int row[RP], lo[TP], hi[TP];
  __device__ __forceinline__ explicit TileOffsets(int lane) {
    const int lr = lane & 31, hf = lane >> 5;
#pragma unroll
    for (int k = 0; k < RP; ++k) row[k] = lr * 8 * U + 8 * ((2 * k + hf) ^ tile_swz(U, lr));
    const int j = lane & 15, gi = lane >> 4;
    const int u = 2 * (gi & 1) + ((j >> 1) & 1), sub = 4 * (j & 1);
    const int rlo = 4 * hf + (j >> 2), rhi = rlo + 8;
#pragma unroll
    for (int nb = 0; nb < TP; ++nb) {
      lo[nb] = rlo * 8 * U + 8 * ((4 * nb + u) ^ tile_swz(U, rlo)) + sub;
      hi[nb] = rhi * 8 * U + 8 * ((4 * nb + u) ^ tile_swz(U, rhi)) + sub;
    }
  }
  // row read of k step kk (compile-time kk: the base index and the added constant fold)
  __device__ __forceinline__ int row_at(int kk) const { return row[kk % RP] + 16 * (kk - kk % RP); }
  __device__ __forceinline__ int lo_at(int nb) const { return lo[nb % TP] + 32 * (nb - nb % TP); }
  __device__ __forceinline__ int hi_at(int nb) const { return hi[nb % TP] + 32 * (nb - nb % TP); }
};

// The periodic bases of TileOffsets made absolute LDS byte addresses of one tile (a stage slot
// changes every step) and opaque: each operand read is then one base register plus an immediate
// offset (k step, column block and the caller's row block), with one VALU add per base per tile
// instead of one or two per read.
template <int U>
struct TileAddr {
  static constexpr int RP = TileOffsets<U>::RP, TP = TileOffsets<U>::TP;
  uint32_t row[RP], lo[TP], hi[TP];
  __device__ __forceinline__ TileAddr(const TileOffsets<U>& o, uint32_t tile) {
#pragma unroll
    for (int k = 0; k < RP; ++k) row[k] = opaque_u32(tile + 2 * o.row[k]);
#pragma unroll
    for (int k = 0; k < TP; ++k) {
      lo[k] = opaque_u32(tile + 2 * o.lo[k]);
      hi[k] = opaque_u32(tile + 2 * o.hi[k]);
    }
  }
  __device__ __forceinline__ uint32_t row_at(int kk) const { return row[kk % RP] + 2 * 16 * (kk - kk % RP); }
  __device__ __forceinline__ uint32_t lo_at(int nb) const { return lo[nb % TP] + 2 * 32 * (nb - nb % TP); }
  __device__ __forceinline__ uint32_t hi_at(int nb) const { return hi[nb % TP] + 2 * 32 * (nb - nb % TP); }
};

// 16-byte LDS reads at a byte address.
__device__ __forceinline__ u32x4 lds_read16_at(uint32_t a) {
  typedef const u32x4 __attribute__((address_space(3))) * lds_u32x4_ptr;
  return *(lds_u32x4_ptr)(size_t)a;
}
__device__ __forceinline__ f32x4 lds_read_f4_at(uint32_t a) {
  typedef const f32x4 __attribute__((address_space(3))) * lds_f32x4_ptr;
  return *(lds_f32x4_ptr)(size_t)a;
}

// 8-element operand from the two transposed chunks at lo and hi.
__device__ __forceinline__ u32x4 lds_tr8(const uint16_t* base, int lo, int hi) {
  const u32x2 a = lds_read_tr16(base + lo);
  const u32x2 b = lds_read_tr16(base + hi);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// 8-element operand of a 32x32x16 MFMA taken from a row-major LDS tile X
// (row stride ld elements) transposed: lane l gets column n0 + l % 32 and the
// rows [R0 + 4 h, R0 + 4 h + 4) followed by [R0 + 8 + 4 h, R0 + 12 + 4 h),
// h = l / 32 -- the k order of a 16-wide group of a 32x32 MFMA result read
// back as an operand.  R0 is a multiple of 16, n0 of 32.  The lane-dependent
// part of the addresses is computed once (TrLane), so every read is the lane
// base plus a compile-time offset.  With SWZ the tile uses the lds_swz layout:
// the two row runs then sit at different swizzles, hence two bases.
struct TrLane {
  int lo, hi;
};
template <bool SWZ>
__device__ __forceinline__ TrLane tr_lane(int ld, int lane) {
  const int j = lane & 15, gi = lane >> 4, h = lane >> 5;
  const int u = 2 * (gi & 1) + ((j >> 1) & 1);   // unit within the 4-unit group at n0
  const int row = 4 * h + (j >> 2);
  const int sub = 4 * (j & 1);
  TrLane t;
  // rows R0 + 4 h + ..: (row >> 2) & 3 == h;  rows R0 + 8 + 4 h + ..: == h + 2
  t.lo = row * ld + 8 * (SWZ ? (u ^ h) : u) + sub;
  t.hi = (row + 8) * ld + 8 * (SWZ ? (u ^ (h + 2)) : u) + sub;
  return t;
}
__device__ __forceinline__ u32x4 lds_operand_tr(const uint16_t* X, const TrLane& t, int ld, int R0, int n0) {
  const uint16_t* p = X + R0 * ld + n0;
  const u32x2 lo = lds_read_tr16(p + t.lo);
  const u32x2 hi = lds_read_tr16(p + t.hi);
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

}  // namespace pope
