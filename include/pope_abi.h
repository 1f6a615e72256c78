/*
 * pope_abi.h -- C ABI of libpope_hip.so, the MI355X (gfx950) PoPE attention path.
 *
 * This is the drop-in boundary below the reference's Python operator layer.
 * Each entry point replaces one launch wrapper of lucidrains/PoPE-pytorch
 * (cited per function).  The Python host layer (pope_amd/hip_pope.py and
 * pope_amd/hip_pope_flash_attn.py) binds these with ctypes and registers them
 * as torch.library ops with autograd.
 *
 * Conventions
 *   - All tensor pointers are DEVICE pointers owned by the caller.  The library
 *     never allocates or frees device memory: scratch space is a caller-owned
 *     workspace whose size pope_workspace_bytes() reports.
 *   - Every entry point returns POPE_OK (0) or a nonzero status; the message of
 *     the last failure on the calling thread is read with pope_last_error().
 *     No C++ exception crosses this boundary.
 *   - Shapes/strides are validated on the host before any HIP call, so argument
 *     errors are testable without a GPU.
 *   - Kernels are enqueued on the caller's stream (a hipStream_t passed as
 *     void*); nothing synchronises the host.  Calls are re-entrant.
 *   - Strides are in ELEMENTS.  The feature (last) dimension must be contiguous.
 */
#ifndef POPE_ABI_H
#define POPE_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define POPE_ABI_VERSION 3

enum pope_dtype { POPE_F32 = 0, POPE_F16 = 1, POPE_BF16 = 2 };

enum pope_status {
  POPE_OK = 0,
  POPE_ERR_INVALID = 1,     /* bad shape / stride / pointer / argument */
  POPE_ERR_UNSUPPORTED = 2, /* valid request the kernels do not cover */
  POPE_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  POPE_ERR_HIP = 4          /* a HIP runtime call failed */
};

enum pope_op { POPE_OP_SIM_FWD = 0, POPE_OP_SIM_BWD = 1, POPE_OP_FLASH_FWD = 2,
               POPE_OP_FLASH_BWD = 3, POPE_OP_FLASH_DECODE = 4, POPE_OP_POLAR_BWD = 5 };

/* pope_desc.flags (flash backward: PREPARED, ZERO_GRADS, DETERMINISTIC; similarity: SPLIT_BF16,
 * DETERMINISTIC; polar transform: COMPLEX, DETERMINISTIC; 0 elsewhere). */
enum pope_flags {
  /* The workspace holds the preparation (expanded K/Q rows, phase tables, key visibility)
   * written by a pope_flash_fwd call with the same descriptor, q, k, freqs, bias and mask,
   * and not modified since: the backward reuses it instead of recomputing it.  The flash
   * forward and backward workspaces have the same size and layout. */
  POPE_FLAG_PREPARED = 1,
  /* dfreqs / dbias are overwritten (cleared by the library before it accumulates into them)
   * instead of accumulated into. */
  POPE_FLAG_ZERO_GRADS = 2,
  /* Similarity forward / backward: the products run on bf16 MFMA with every fp32 operand split
   * into hi + lo bf16 halves (three products per pair, 16 significant operand bits, fp32
   * accumulation) -- the counterpart of the reference's default allow_tf32=True (TF32 keeps 10
   * bits, triton_pope.py:63,145,224).  Without it the products are true fp32 MFMA. */
  POPE_FLAG_SPLIT_BF16 = 4,
  /* Polar transform: q_hat / k_hat rows are D (re, im) fp32 pairs, the complex64 layout of the
   * reference's return_complex=True output (torch.polar, pope.py:49-51,66-67,74-75): the rotated
   * dims as (a cos, a sin), pass-through dim d as (x_d, 0). */
  POPE_FLAG_COMPLEX = 8,
  /* Backward of the flash attention, the similarity and the polar transform: dfreqs and dbias
   * are bitwise reproducible from call to call.  Every phase derivative is written once to the
   * workspace (which grows by (B Hk Nk + B Hq Nq) R + 64 Hb R floats) and summed in a fixed
   * order, instead of fp32 atomics whose order varies.  The other gradients are deterministic
   * either way. */
  POPE_FLAG_DETERMINISTIC = 16
};

/*
 * Problem descriptor shared by every entry point.
 *
 * q: (B, Hq, Nq, D)   k, v: (B, Hk, Nk, D)   o / dq / do like q, dk / dv like k,
 * addressed as x[b*s[0] + h*s[1] + n*s[2] + d].  Query head h reads kv head
 * h % Hk (the reference's 'b h ... -> b (g h) ...' repeat, attention.py:44-45).
 * freqs: rows n < Nk of an (N, R) / (B, N, R) / per-head table, addressed as
 * f[b*f_s[0] + h*f_s[1] + n*f_s[2] + r] (0 strides broadcast); the key phase is
 * freqs[j] + bias, the query phase freqs[Nk - Nq + i] (right-aligned,
 * pope.py:64, triton_pope_flash_attn.py:54).  R == 0 means no PoPE (plain
 * attention / plain q k^T).  D and R are multiples of 8 (rows move in 16-byte
 * chunks); flash takes D <= 128, the similarity D <= 512.  The reference takes
 * any D and R (triton_pope.py:58-60, triton_pope_flash_attn.py:44,252); other
 * shapes are padded by the caller first: rotated dims with a value whose
 * softplus is 0 (-1e4), pass-through dims, v, freqs and bias with zeros (the
 * Python layer does this, pope_amd/_pad.py).  bias: (Hb, R) with Hb in {1, Hk}, row stride
 * bias_sh (0 when Hb == 1); it must already be clamped to [-2*pi, 0]
 * (pope.py:145).  mask: (B, Nk) bytes, nonzero = keep (attention.py:129-131).
 */
typedef struct pope_desc {
  int32_t B, Hq, Hk, Nq, Nk, D, R;
  int32_t dtype;          /* enum pope_dtype of q, k, v, o and their grads */
  int32_t causal;         /* top-left causal: key j visible to query i iff j <= i */
  float softmax_scale;    /* flash only; the reference default is D ** -0.5 */
  int32_t flags;          /* enum pope_flags */
  int64_t q_s[3], k_s[3], v_s[3], o_s[3];
  int64_t do_s[3], dq_s[3], dk_s[3], dv_s[3];
  int64_t sim_s[3];       /* similarity output (b, h, i); column stride 1 */
  int64_t f_s[3];         /* freqs (b, h, n) strides */
  int64_t df_s[3];        /* dfreqs (b, h, n) strides; fp32 accumulation target */
  int64_t bias_sh;        /* bias / dbias row stride */
  int64_t mask_sb;        /* mask batch stride in bytes */
} pope_desc;

/* Version of this header the library was built from. */
int pope_abi_version(void);

/* Copies the last error message of the calling thread (NUL-terminated). */
int pope_last_error(char* buf, size_t n);

/* Bytes of caller-owned device workspace an operation needs (no counterpart in
 * the reference, whose launch wrappers allocate scratch through torch:
 * triton_pope.py:267-272,297-300; triton_pope_flash_attn.py:288,358-359). */
int pope_workspace_bytes(int op, const pope_desc* desc, size_t* bytes);

/*
 * Fused PoPE similarity forward, fp32 MFMA:  sim[b,h,i,j] (unscaled).
 * Replaces PoPESimilarityFunction.forward + _fwd_kernel launch
 * (triton_pope.py:260-288; kernel :28-83).  dtype: POPE_F32 (inputs and sim).
 */
int pope_sim_fwd(const pope_desc* desc, const void* q, const void* k, const float* freqs,
                 const float* bias, void* sim, void* workspace, size_t workspace_bytes,
                 void* stream);

/*
 * Fused PoPE similarity backward.  dsim has the sim layout (sim_s).  dq, dk are
 * written (not accumulated).  dfreqs (fp32, df_s strides) and dbias (fp32, Hb
 * rows, bias_sh) are ACCUMULATED into and may be NULL (caller zeroes), or
 * overwritten with POPE_FLAG_ZERO_GRADS: dfreqs rows n < Nk, every dbias row.
 * Replaces PoPESimilarityFunction.backward (triton_pope.py:291-362; kernels
 * _bwd_kernel_dqk_df :85-194 and _bwd_kernel_dbias_optimized :196-256).
 */
int pope_sim_bwd(const pope_desc* desc, const void* dsim, const void* q, const void* k,
                 const float* freqs, const float* bias, void* dq, void* dk, float* dfreqs,
                 float* dbias, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Flash attention forward with PoPE fused (online softmax, top-left causal,
 * key-padding mask).  Writes o (dtype) and lse (fp32, (B, Hq, Nq) contiguous,
 * natural log, -inf for fully masked rows).  freqs/bias may be NULL when R == 0,
 * mask may be NULL.  dtype: POPE_BF16 or POPE_F16.
 * Replaces flash_attn_forward (triton_pope_flash_attn.py:222-271; kernel :23-117).
 */
int pope_flash_fwd(const pope_desc* desc, const void* q, const void* k, const void* v,
                   const float* freqs, const float* bias, const uint8_t* mask, void* o,
                   float* lse, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Flash attention backward with PoPE.  dq, dk, dv are written (not accumulated);
 * dfreqs / dbias are fp32 and ACCUMULATED into (caller zeroes; NULL = not wanted),
 * or overwritten with POPE_FLAG_ZERO_GRADS.  With POPE_FLAG_PREPARED the workspace of
 * the matching pope_flash_fwd call is reused as is.
 * Replaces flash_attn_backward (triton_pope_flash_attn.py:273-335; kernels
 * _bwd_preprocess :119-130 and _bwd_kernel :132-218).
 */
int pope_flash_bwd(const pope_desc* desc, const void* dout, const void* q, const void* k,
                   const void* v, const void* o, const float* lse, const float* freqs,
                   const float* bias, const uint8_t* mask, void* dq, void* dk, void* dv,
                   float* dfreqs, float* dbias, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * Bandwidth-bound forward for a single non-causal query row against a long KV
 * cache (decode): split-K over the keys plus an LSE merge.  Same contract as
 * pope_flash_fwd; returns
 * POPE_ERR_UNSUPPORTED (callers then use pope_flash_fwd) for: Nq != 1; causal; head
 * dim above 128; per-head freqs tables (f_s[1] != 0); no power-of-two group of the
 * query heads (dividing Hq) with at most 4096 query-weight words (group heads x head
 * dim: the weights are staged in LDS, one group per workgroup); freqs rows that are not 16-byte
 * aligned (pointer, f_s[0] or f_s[2] not a multiple of 4 floats); K / V row offsets
 * within a (batch, head) beyond 32 bits.  Replaces flash_attn_forward at
 * seqlen_q = 1 (triton_pope_flash_attn.py:222-271 with grid (1, B*H)).
 */
int pope_flash_decode(const pope_desc* desc, const void* q, const void* k, const void* v,
                      const float* freqs, const float* bias, const uint8_t* mask, void* o,
                      float* lse, void* workspace, size_t workspace_bytes, void* stream);

/*
 * pope_flash_decode without a workspace argument and without any allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The split partials live in a
 * 16 MiB device array of the library (one per GPU, held until the process ends); a call whose
 * partials need more (pope_workspace_bytes(POPE_OP_FLASH_DECODE) above 16 MiB, i.e. more batch
 * rows x query heads x splits) fails with POPE_ERR_WORKSPACE.  Calls that overlap on one GPU
 * share that array and race: serialise them (one stream, or events).  Same results as
 * pope_flash_decode.
 */
int pope_flash_decode_noalloc(const pope_desc* desc, const void* q, const void* k, const void* v,
                              const float* freqs, const float* bias, const uint8_t* mask, void* o,
                              float* lse, void* stream);

/*
 * Materialising polar transform: q_hat, k_hat = apply_pope_to_qk(pos, q, k) with the default
 * softplus magnitude (pope.py:30-86).  q (B, Hq, Nq, D), k (B, Hk, Nk, D) in dtype (F32, F16 or
 * BF16, q_s / k_s strides, multiples of 4); q_hat (B, Hq, Nq, D + R), k_hat (B, Hk, Nk, D + R)
 * are contiguous fp32 (the reference's dtype promotion against fp32 cos / sin, :69-70): the
 * first 2R columns interleave (a cos, a sin) per rotated dim with a = softplus rounded to dtype
 * (:60), the last D - R are the raw pass-through dims (:82-84).  Query rows take the phases
 * freqs[Nk - Nq + i] (:64), key rows fl(freqs[j] + bias[h]) (:56); bias is used as given.
 * With POPE_FLAG_COMPLEX (the only flag it takes) the rows are (B, H, N, 2 D) instead: complex64
 * pairs, pass-through dims as (x, 0) (return_complex, :49-51,66-67,74-75).
 */
int pope_polar_fwd(const pope_desc* desc, const void* q, const void* k, const float* freqs, const float* bias,
                   float* q_hat, float* k_hat, void* stream);

/*
 * Backward of pope_polar_fwd: dq_hat / dk_hat are contiguous fp32 gradients of its outputs;
 * dq, dk (dtype, dq_s / dk_s strides) are written; dfreqs (fp32, df_s strides) and dbias (fp32,
 * bias rows bias_sh) are ACCUMULATED into (NULL = not wanted).  The autograd backward of the
 * reference's torch ops (pope.py:30-86).  With POPE_FLAG_COMPLEX the gradients come in the
 * complex layout of the forward (a pass-through dim takes sign(x) times the real part of its
 * pair's gradient: the backward of torch.polar(x, 0) the reference builds it with).  The
 * workspace (pope_workspace_bytes(POPE_OP_POLAR_BWD)) is empty unless POPE_FLAG_DETERMINISTIC.
 */
int pope_polar_bwd(const pope_desc* desc, const float* dq_hat, const float* dk_hat, const void* q, const void* k,
                   const float* freqs, const float* bias, void* dq, void* dk, float* dfreqs, float* dbias,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-kernel timing.  No counterpart in the reference (its tests print only
 * parity diffs, tests/test_flash_attn.py:61,109).  While enabled, every kernel
 * launch of the library carries a pair of hipEvents that its dispatch stamps with
 * the kernel's own start and end (hipExtLaunchKernel), on the stream the kernel
 * runs on.  pope_profile_read waits for the recorded events
 * and writes one line per kernel name, "name count total_ms min_ms max_ms",
 * cumulative since the last pope_profile_reset.  Used by bench.py to time the
 * dominant kernel on its own stream.
 */
int pope_profile_enable(int on);
int pope_profile_read(char* buf, size_t n);
int pope_profile_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* POPE_ABI_H */
