// Kernel parameter blocks and launchers shared between the kernels and the C ABI.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pope {

// Per-kernel timing (profile.cpp).  prof_begin returns -1 when profiling is off, else a token
// and the event pair the launch records its own start / end timestamps into.
int prof_begin(const char* name, hipEvent_t* start, hipEvent_t* stop);
void prof_cancel(int token);
void prof_enable(int on);
int prof_read(char* buf, size_t n);
void prof_reset();

// Launches `kernel`; when profiling is on, the dispatch itself records its start and end
// timestamps into a pair of events (hipExtLaunchKernel), so the elapsed time is the kernel's
// execution alone, as a kernel trace reports it.
template <typename... KArgs, typename... Args>
hipError_t launch_named(const char* name, void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t s,
                        Args... args) {
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  const int t = prof_begin(name, &ev0, &ev1);
  if (t < 0) {
    hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
    return hipGetLastError();
  }
  hipExtLaunchKernelGGL(kernel, grid, block, 0, s, ev0, ev1, 0u, args...);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) prof_cancel(t);
  return e;
}

// cos/sin of the phase table: tab[bt*t_sb + ht*t_sh + n*R + d] = (cos, sin) of
// F[n, d] (+ bias[ht, d] when a bias is folded in), for n < rows.
struct TableParams {
  const float* freqs; int64_t f_sb, f_sh, f_sn;
  const float* bias; int64_t bias_sh;  // may be null
  int Bt, Ht, rows, R;
  float2* out;               // fp32 (cos, sin), or
  uint32_t* out16;           // fp16 (cos, sin) pairs packed per 32-bit word when non-null
};
hipError_t launch_phase_table(const TableParams& p, hipStream_t s);

// Shared preparation of the flash forward and backward (flash_prep.hip, one launch), written
// into the caller's workspace once per forward call and reused by the backward: K_hat and the
// pre-scaled Q_hat rows, cos/sin(F) rows n < Nk (fp32 pairs), cos/sin(bias) per (bias row, dim),
// the key visibility words and 1 + last visible key per batch.
// The expanded rows (16-bit, EP columns, zero past E and past Nq / Nk) are
//   K_hat[b, hk, j] = [c cos F_j | c sin F_j | k_rest],                c = softplus(k_j)
//   Q_hat[b, h, i]  = s [a cos(F_i' - bias) | a sin(F_i' - bias) | q_rest],  a = softplus(q_i),
// F_i' = F[Nk - Nq + i] and s = softmax_scale * log2(e), so Q_hat K_hat^T is the score in log2
// units.  The learned bias sits on the query side: cos(phi - (F_j + b)) = cos((phi - b) - F_j).
struct FlashPrep {
  const uint16_t* q; const uint16_t* k;
  const float* freqs; const float* bias; const uint8_t* mask;
  float2* table;             // (Bt, Ht, Nk, R)
  float2* btab;              // (Hb, R)
  uint16_t* qh;              // (B, Hq, NqP, EP)
  uint16_t* kh;              // (B, Hk, NkP, EP)
  uint64_t* mwords;          // (B, NW): bit j of word w <=> key 64 w + j < Nk and unmasked
  int* kend;                 // (B)
  int B, Hq, Hk, Nq, Nk, D, R, EP, NqP, NkP, NW, Bt, Ht, Hb, has_mask;
  float qscale;
  int64_t q_s[3], k_s[3], f_s[3];
  int64_t bias_sh, mask_sb, t_sb, t_sh;
};
// dtype: 1 = f16, 2 = bf16.
hipError_t launch_flash_prep(const FlashPrep& p, int dtype, hipStream_t s);

struct FlashFwdParams {
  const uint16_t* qh; const uint16_t* kh; const uint16_t* v;   // Q_hat, K_hat of FlashPrep
  const uint64_t* mwords; const int* kend;
  uint16_t* o; float* lse;
  int B, Hq, Hk, Nq, Nk, D, EP, DV, NqP, NkP, NW, causal, nqb;
  int64_t v_s[3], o_s[3];
};
// Returns hipErrorInvalidValue for an uncovered (EP, DV) shape.
hipError_t launch_flash_fwd(const FlashFwdParams& p, int dtype, hipStream_t s);

struct FlashBwdParams {
  const uint16_t* q; const uint16_t* k; const uint16_t* v; const uint16_t* o; const uint16_t* dout;
  const float* lse; const uint8_t* mask;
  const float2* table;       // cos/sin(F[b, h, n, d]) for n < Nk (FlashPrep::table)
  const float2* btab;        // cos/sin(bias) (FlashPrep::btab)
  uint16_t* dq; uint16_t* dk; uint16_t* dv;
  float* dfreqs; float* dbias;
  // workspace (FlashPrep): expanded rows, zero past Nq / Nk and past E
  const uint16_t* qh;        // (B, Hq, NqP, EP)  Q_hat * softmax_scale * log2(e)
  const uint16_t* kh;        // (B, Hk, NkP, EP)  K_hat
  float* nl; float* nd;      // (B, Hq, NqP)      -lse * log2(e) and -rowsum(O * dO); rows past Nq and
                             //                   rows with every key masked carry -inf in nl
  const uint64_t* mwords; const int* kend;   // key visibility (FlashPrep)
  int NW;
  int B, Hq, Hk, Nq, Nk, D, R, E, EP, DV, NqP, NkP, causal, has_mask;
  int Bt, Ht, Hb;            // extents of the cos/sin table and of the bias rows
  int zero_grads;            // clear dfreqs / dbias before accumulating
  float* kpart; float* qpart;   // deterministic mode: per-row phase derivatives (PhaseGradParams), else null
  int n_kv_jobs, interleave; // dK/dV jobs of the fused launch; 1 = pair dK/dV and dQ jobs by cost
  float scale;
  int64_t q_s[3], k_s[3], v_s[3], o_s[3], do_s[3], dq_s[3], dk_s[3], dv_s[3], df_s[3];
  int64_t bias_sh, mask_sb, t_sb, t_sh;
};
hipError_t launch_flash_bwd(const FlashBwdParams& p, int dtype, hipStream_t s);
// The backward's row terms alone (-lse log2 e and -delta per query row; dfreqs / dbias cleared
// with zero_grads): the wide path's first launch.
hipError_t launch_flash_bwd_delta(const FlashBwdParams& p, int dtype, hipStream_t s);

// Wide heads (flash_wide.hip): DV = 256 and EP in {256, 384, 512}.  The backward takes two fp32
// workspaces for the raw expanded-row gradients, wk (B, Hk, NkP, EP) and wq (B, Hq, NqP, EP).
bool flash_wide_shape(int EP, int DV);
hipError_t launch_flash_wide_fwd(const FlashFwdParams& p, int dtype, hipStream_t s);
hipError_t launch_flash_wide_bwd(const FlashBwdParams& p, float* wk, float* wq, int dtype, hipStream_t s);

struct SimParams {
  const float* q; const float* k; const float* dsim; float* sim;
  const float* freqs; const float* bias;
  const float2* ktab;        // cos/sin(F[j] + bias[hk]) per (bt, hk) for keys
  const float2* qtab;        // cos/sin(F[n]) per bt, rows n < Nk (queries use n = q_off + i)
  float* dq; float* dk; float* dfreqs; float* dbias;
  int B, Hq, Hk, Nq, Nk, D, R, E, EP;
  int g_vec;                 // dsim rows are 16-byte aligned: 4-wide loads allowed
  float* kpart; float* qpart;   // deterministic mode: per-row phase derivatives (PhaseGradParams), else null
  int zero_grads;            // backward: the first launch clears dfreqs (Bt, Ht, n < Nk) and dbias (Hb)
  int Bt, Ht, Hb;            // extents of dfreqs / dbias (1 where freqs / bias broadcast)
  int64_t q_s[3], k_s[3], sim_s[3], dq_s[3], dk_s[3], f_s[3], df_s[3];
  int64_t bias_sh, kt_sb, kt_sh, qt_sb, qt_sh;
};
hipError_t launch_sim_fwd(const SimParams& p, hipStream_t s);
// U: (B, Hq, Nq, EP) and W: (B, Hk, Nk, EP) fp32 workspace.
hipError_t launch_sim_bwd_ws(const SimParams& p, float* U, float* W, hipStream_t s);
// Chain rule of the polar transform on U (queries) and W (keys) (sim.hip); U2 / W2 are second
// partial sums added to them, or null.
hipError_t launch_sim_finalize(const SimParams& p, const float* U, const float* U2, const float* W, const float* W2,
                               hipStream_t s);

// Split-bf16 similarity (sim_split.hip): hi / lo bf16 planes of Q_hat and K_hat, rows padded
// to 128, row-major (heads, NP, EP) for the forward or transposed (heads, EP, NP) for the
// backward.
struct SimSplit {
  uint16_t* qh; uint16_t* ql; uint16_t* kh; uint16_t* kl;
  int NqP, NkP;
  float* U2; float* W2;      // backward: second partial sums of U and W (split reduction)
};
hipError_t launch_sim_split_fwd(const SimParams& p, const SimSplit& sp, hipStream_t s);
hipError_t launch_sim_split_bwd(const SimParams& p, const SimSplit& sp, float* U, float* W, hipStream_t s);

// Materialising polar transform (polar.hip): q_hat / k_hat fp32 rows (heads, N, D + R).
struct PolarParams {
  const void* q; const void* k; const float* freqs; const float* bias;
  float* qh; float* kh;                 // forward outputs
  const float* gq; const float* gk;     // backward: gradients of q_hat / k_hat
  void* dq; void* dk; float* dfreqs; float* dbias;
  int B, Hq, Hk, Nq, Nk, D, R;
  int cplx;                             // rows of D (re, im) pairs (complex64 layout) instead of D + R
  float* kpart; float* qpart;           // deterministic mode: per-row phase derivatives, else null
  int64_t q_s[3], k_s[3], dq_s[3], dk_s[3], f_s[3], df_s[3];
  int64_t bias_sh;
};
// dtype: 0 fp32, 1 fp16, 2 bf16 (of q, k, dq, dk)
hipError_t launch_polar(const PolarParams& p, int dtype, bool bwd, hipStream_t s);

// Deterministic phase gradients (phase_grad.hip): the backward kernels write every key-side phase
// derivative dpsi once to kpart (B, Hk, Nk, R) and every query-side one dphi to qpart (B, Hq, Nq, R)
// (query row i <-> phase row Nk - Nq + i); these sums add them in a fixed order into dfreqs
// (Bt, Ht, Nk, R strides df_s) and dbias (Hb rows, bias_sh): `overwrite` replaces their contents,
// otherwise the sums are added to them.  bslices: phase_grad_slices(Hb, R) floats of scratch.
struct PhaseGradParams {
  const float* kpart; const float* qpart;   // qpart may be null (no query-side derivatives)
  float* dfreqs; float* dbias;              // null: not wanted
  float* bslices;
  int B, Hq, Hk, Nq, Nk, R, Bt, Ht, Hb, overwrite;
  int64_t df_s[3];
  int64_t bias_sh;
};
size_t phase_grad_slices(int Hb, int R);
hipError_t launch_phase_grad_reduce(const PhaseGradParams& p, hipStream_t s);

struct DecodeParams {
  const uint16_t* q; const uint16_t* k; const uint16_t* v;
  const float* freqs; const float* bias; const uint8_t* mask;   // freqs rows 16-byte aligned
  uint16_t* o; float* lse;
  float* part_o; float* part_ml;   // split-K partials (B*Hq*Nq, splits, D) and (.., splits, 2)
  int B, Hq, Hk, Nq, Nk, D, R, causal, has_mask, splits, keys_per_split;
  int hgroups;                     // query-head groups per split (set by launch_flash_decode)
  float scale_log2;
  int64_t q_s[3], k_s[3], v_s[3], o_s[3], f_s[3];
  int64_t bias_sh, mask_sb, t_sb, t_sh;
};
// Keys per split of the decode kernel at head dim D.  launch_flash_decode returns
// hipErrorInvalidValue for shapes the kernel does not cover (Nq != 1, causal, D > 128, per-head
// freqs, decode_head_groups(Hq, D) == 0).
int decode_split_keys(int D);
// Query-head groups per split workgroup: the fewest (a power of two dividing Hq) whose heads'
// query weights fit the kernel's 4096-word LDS array, or 0 when none does.
int decode_head_groups(int Hq, int D);
// The decode's scratch array on the current device (its device address, looked up once per
// device): kDecodeScratchBytes, for the entry point that allocates nothing.
constexpr size_t kDecodeScratchBytes = (size_t)16 << 20;
hipError_t decode_scratch(void** ptr);
hipError_t launch_flash_decode(const DecodeParams& p, int dtype, hipStream_t s);

}  // namespace pope
