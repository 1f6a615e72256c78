"""Flash attention with PoPE on the HIP kernels of libpope_hip.so.

Operator mirror of the reference's ``PoPE_pytorch/triton_pope_flash_attn.py``:
``flash_attn_forward`` (:222-271), ``flash_attn_backward`` (:273-335),
``FlashAttnFunction`` (:337-362) and ``flash_attn`` (:364-373) keep their names,
arguments, (batch, seq, heads, dim) layout and return values.  Underneath, two
``torch.library`` custom ops carry the work:

  pope_amd::flash_fwd(q, k, v, freqs?, bias?, mask?, causal, scale) -> (o, lse)
  pope_amd::flash_bwd(do, q, k, v, o, lse, freqs?, bias?, mask?, causal, scale,
                      need_dfreqs, need_dbias) -> (dq, dk, dv, dfreqs, dbias)

with ``flash_fwd`` differentiable through ``register_autograd``.  Eager calls of
``flash_attn`` / ``flash_attn_head_first`` run the same forward and backward through a
plain ``autograd.Function`` (no custom-op dispatch, which costs more host time than a
launch); torch.compile tracing records the ops.  The ops take
head-first logical views (B, H, N, D) with any batch/head/seq strides and a unit
feature stride, so the (b n h d) <-> (b h n d) permutes of the reference cost no
copies.  Query head h reads kv head h % Hk (the reference's torch-path GQA
mapping, attention.py:118-120; the reference's fused kernel has no GQA).

Differences from the reference kernels, by design:
  * dq is accumulated in fp32 (the reference adds bf16 atomics, :215,358);
  * the backward skips key/query tiles past the causal diagonal (:167 visits all);
  * out-of-range keys are always masked (:152-199 leaves them in when the call is
    non-causal, unmasked and Nk % 32 != 0);
  * fp32 inputs run the fp16 MFMA kernels on fp16-rounded q, k, v, 10 significant bits (the reference
    runs tl.dot at TF32 for fp32, which is likewise a reduced-precision product).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from ._pad import pad_last, pad_plan, pad_qk, unpad_qk

_MFMA_DTYPES = (torch.bfloat16, torch.float16)


def exists(v):
    return v is not None


def _freqs_strides(freqs: Tensor, head_first: bool = True) -> tuple:
    """(b, h, n) element strides of a freqs table (r stride must be 1).

    2-D (N, R): shared; 3-D (B, N, R): per batch; 4-D: (B, H, N, R) head-first
    or (B, N, H, R) when the caller works in (batch, seq, heads) layout
    (triton_pope_flash_attn.py:237-245)."""
    # a batch or head extent of 1 broadcasts: stride 0, so the library sees one shared table
    s = [0 if n == 1 else st for n, st in zip(freqs.shape, freqs.stride())]
    if freqs.ndim == 2:
        return (0, 0, s[0])
    if freqs.ndim == 3:
        return (s[0], 0, s[1])
    if freqs.ndim == 4:
        return (s[0], s[1], s[2]) if head_first else (s[0], s[2], s[1])
    raise ValueError(f"freqs must be 2-D, 3-D or 4-D, got shape {tuple(freqs.shape)}")


def _prep_pope(freqs: Optional[Tensor], bias: Optional[Tensor]):
    if freqs is None or bias is None:
        return None, None
    if freqs.dtype != torch.float32:
        freqs = freqs.float()
    # rows of 16-byte vectors: unit feature stride, row / batch / head strides and the view's
    # offset in whole 4-float units (storage_offset, not data_ptr, so fake tensors decide alike)
    # (rotate dims that are not multiples of 8 are padded into a fresh table later; under
    # torch.compile tracing the offset is not inspected, and the forward copies a misaligned
    # table itself where the decode kernel needs it)
    misaligned = freqs.shape[-1] % 8 == 0 and any(s % 4 for s in freqs.stride()[:-1])
    if not torch.compiler.is_compiling() and freqs.shape[-1] % 8 == 0:
        misaligned = misaligned or freqs.storage_offset() % 4 != 0
    if freqs.stride(-1) != 1 or misaligned:
        freqs = freqs.clone(memory_format=torch.contiguous_format)
    if bias.dtype != torch.float32:
        bias = bias.float()
    if bias.ndim == 1:
        bias = bias.unsqueeze(0)
    if bias.stride(-1) != 1:
        bias = bias.contiguous()
    return freqs, bias


def _prep_mask(mask: Optional[Tensor], B: int):
    if mask is None:
        return None
    if mask.dtype != torch.bool:
        mask = mask.bool()
    if mask.ndim != 2:
        raise ValueError(f"mask must be (batch, seq_k), got {tuple(mask.shape)}")
    if mask.shape[0] == 1 and B > 1:
        mask = mask.expand(B, mask.shape[1])
    if mask.stride(-1) != 1:
        mask = mask.contiguous()
    return mask


def _unit_feature(t: Tensor) -> Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _desc(q, k, freqs, bias, causal, scale, head_first_freqs=True) -> _lib.PopeDesc:
    B, Hq, Nq, D = q.shape
    Hk, Nk = k.shape[1], k.shape[2]
    d = _lib.PopeDesc()
    d.B, d.Hq, d.Hk, d.Nq, d.Nk, d.D = B, Hq, Hk, Nq, Nk, D
    d.R = freqs.shape[-1] if exists(freqs) else 0
    d.dtype = _lib.dtype_code(q.dtype)
    d.causal = 1 if causal else 0
    d.softmax_scale = float(scale)
    if exists(freqs):
        d.f_s[:] = _freqs_strides(freqs, head_first_freqs)
        d.bias_sh = bias.stride(0) if bias.shape[0] > 1 else 0
    return d


def _check_pope_shapes(q, k, freqs, bias):
    B, Hq, Nq, D = q.shape
    if k.shape[0] != B or k.shape[3] != D or Hq % k.shape[1] != 0:
        raise ValueError(f"incompatible q {tuple(q.shape)} and k {tuple(k.shape)}")
    if exists(freqs):
        R = freqs.shape[-1]
        if R > D:
            raise AssertionError(f"rotate dim {R} exceeds head dim {D}")
        if freqs.shape[-2] < k.shape[2]:
            raise ValueError(f"freqs has {freqs.shape[-2]} positions, keys need {k.shape[2]}")
        if bias.shape[-1] != R or bias.shape[0] not in (1, k.shape[1]):
            raise ValueError(f"bias {tuple(bias.shape)} must be (1 or {k.shape[1]}, {R})")


def _check_views(q, k, v, mask, lse=None):
    """Shapes the kernels index by but the descriptor does not carry.  Cheap tuple compares:
    run on every call, not only when a call plan is built."""
    if v.shape != k.shape:
        raise ValueError(f"v {tuple(v.shape)} must match k {tuple(k.shape)}")
    if exists(mask) and tuple(mask.shape) != (q.shape[0], k.shape[2]):
        raise ValueError(f"mask {tuple(mask.shape)} must be (batch, seq_k) = {(q.shape[0], k.shape[2])}")
    if exists(lse) and tuple(lse.shape) != tuple(q.shape[:3]):
        raise ValueError(f"lse {tuple(lse.shape)} must be {tuple(q.shape[:3])}")


def _check_dtypes(q, *others):
    """The descriptor carries one element type, q's: every other 16-bit operand must match it."""
    for t in others:
        if t.dtype != q.dtype:
            raise TypeError(f"pope_amd flash: operand of dtype {t.dtype} next to q of dtype {q.dtype}")


_FP16_MAX = 65504.0


def _check_fp16_range(*ts):
    """fp32 flash inputs run on fp16 operands: a finite value beyond fp16's range would become inf
    silently, so such inputs raise instead.  The check reads one flag back to the host (fp32 flash
    is the compatibility path; the bf16 / fp16 paths never synchronise); under torch.compile
    tracing it is skipped."""
    if torch.compiler.is_compiling():
        return
    bad = torch.zeros((), dtype=torch.bool, device=ts[0].device)
    for t in ts:
        bad |= ((t.abs() > _FP16_MAX) & t.isfinite()).any()
    if bool(bad):
        raise ValueError("pope_amd flash: fp32 q / k / v run on fp16 operands (10-bit mantissa, as the "
                         "reference's TF32 products) and must stay within fp16's range |x| <= 65504; "
                         "scale the inputs or pass bf16")


_INT32_MAX = 2 ** 31 - 1
_DECODE_QUERY_WORDS = 4096   # query-weight words a decode workgroup stages in LDS


def _decode_head_groups(Hq: int, D: int) -> int:
    """decode_head_groups() of the library: the fewest power-of-two groups of the query heads
    whose query weights fit the decode workgroup's LDS array, or 0 when none does."""
    g = 1
    while g <= Hq:
        if Hq % g == 0 and (Hq // g) * D <= _DECODE_QUERY_WORDS:
            return g
        g *= 2
    return 0


def _decode_eligible(q, k, v, freqs, causal) -> bool:
    """Whether the forward runs the split-K decode kernel (pope_flash_decode): one non-causal query
    row against a cache of at least 1024 keys, within the decode kernel's head-dim and 32-bit index
    limits.  The forward op and its fake implementation both decide with this predicate, so the
    workspace they return has the same size (empty for decode)."""
    B, Hq, Nq, D = q.shape
    Nk = k.shape[2]
    R = freqs.shape[-1] if exists(freqs) else 0
    if Nq != 1 or causal or Nk < 1024 or D > 128:
        return False
    if _decode_head_groups(Hq, D) == 0:
        return False   # a workgroup stages its group's query weights in LDS
    if R and (_freqs_strides(freqs)[1] != 0 or any(st % 4 for st in _freqs_strides(freqs))):
        return False   # per-head tables, or rows that are not whole 16-byte vectors
    return (Nk - 1) * max(k.stride(2), v.stride(2)) + D < _INT32_MAX


# ------------------------------------------------------------------ call plans
#
# A plan is the filled descriptor and workspace size for one combination of shapes,
# strides, dtype and flags.  Building one costs a few dozen ctypes field writes and a
# library query; a training loop repeats the same few combinations, so plans are
# cached by a key of everything the descriptor is made from.  The library only reads
# the descriptor, so one cached instance serves every call with that key.

_PLANS: dict = {}
_PLANS_MAX = 1024


def _plan(key, build):
    p = _PLANS.get(key)
    if p is None:
        if len(_PLANS) >= _PLANS_MAX:
            _PLANS.clear()
        p = _PLANS[key] = build()
    return p


def _opt_key(t):
    return None if t is None else (t.shape, t.stride())


def _stream(t: Tensor) -> int:
    return torch._C._cuda_getCurrentRawStream(t.get_device())


def _data(t):
    return None if t is None else t.data_ptr()


def _fwd_ws_bytes(d, deterministic: int) -> int:
    """The forward's workspace: the preparation the backward reuses and, under deterministic mode,
    the backward's phase-derivative region after it, so that the backward takes the buffer as is."""
    if not deterministic:
        return _lib.workspace_bytes(_lib.OP_FLASH_FWD, d)
    dd = _lib.PopeDesc.from_buffer_copy(d)
    dd.flags = deterministic
    return _lib.workspace_bytes(_lib.OP_FLASH_BWD, dd)


def _fwd_impl(q, k, v, freqs, bias, mask, causal, softmax_scale):
    q, k, v = _unit_feature(q), _unit_feature(k), _unit_feature(v)
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    _check_views(q, k, v, mask)
    deterministic = _lib.deterministic_flag()
    key = ("fwd", deterministic, q.shape, q.stride(), k.shape, k.stride(), v.shape, v.stride(), o.stride(),
           q.dtype, k.dtype, v.dtype, causal, softmax_scale, _opt_key(freqs), _opt_key(bias), _opt_key(mask))

    def build():
        _check_dtypes(q, k, v)
        _check_pope_shapes(q, k, freqs, bias)
        d = _desc(q, k, freqs, bias, causal, softmax_scale)
        d.q_s[:], d.k_s[:], d.v_s[:] = _lib.strides3(q), _lib.strides3(k), _lib.strides3(v)
        d.o_s[:] = _lib.strides3(o)
        if exists(mask):
            d.mask_sb = mask.stride(0)
        # one non-causal query row against a long cache: the split-K decode kernel
        decode = _decode_eligible(q, k, v, freqs, causal)
        dec_bytes = _lib.workspace_bytes(_lib.OP_FLASH_DECODE, d) if decode else -1
        return d, dec_bytes, _fwd_ws_bytes(d, deterministic)

    d, dec_bytes, fwd_bytes = _plan(key, build)
    L = _lib.lib()
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), _data(freqs), _data(bias), _data(mask),
            o.data_ptr(), lse.data_ptr())
    stream = _stream(q)
    if dec_bytes >= 0:
        if exists(freqs) and freqs.data_ptr() % 16:
            # a table in memory torch did not allocate (its base is not 16-byte aligned): run on an
            # aligned dense copy, with a descriptor for the copy's strides
            freqs = freqs.clone(memory_format=torch.contiguous_format)
            args = args[:3] + (freqs.data_ptr(),) + args[4:]
            d = _lib.PopeDesc.from_buffer_copy(d)
            d.f_s[:] = _freqs_strides(freqs)
        dws = torch.empty(dec_bytes, dtype=torch.uint8, device=q.device) if dec_bytes else None
        _lib.check(L.pope_flash_decode(ctypes.byref(d), *args, _data(dws), dec_bytes, stream), "flash decode")
        return o, lse, q.new_empty(0, dtype=torch.uint8)
    # torch's caching allocator returns 512-byte aligned blocks
    ws = torch.empty(fwd_bytes, dtype=torch.uint8, device=q.device)
    _lib.check(L.pope_flash_fwd(ctypes.byref(d), *args, ws.data_ptr(), fwd_bytes, stream), "flash forward")
    return o, lse, ws


# whether the last backward reused its forward's preparation (read by tests)
_LAST_BWD_PREPARED = False

# whether the forward's workspace is kept for the backward (set_flash_workspace_reuse)
_REUSE_FWD_WORKSPACE = True


def set_flash_workspace_reuse(enabled: bool) -> None:
    """Keep the flash forward's workspace (the expanded K_hat / Q_hat rows, phase tables and key
    words of its preparation) alive for the backward, which then skips the preparation (the
    default); or let it go after the forward, so that no memory beyond the reference's saved
    tensors is held between forward and backward (25.2 MB at B2 H8 N4096 D64 R32) and the
    backward repeats the preparation (about 13 us there).  No counterpart in the reference."""
    global _REUSE_FWD_WORKSPACE
    _REUSE_FWD_WORKSPACE = bool(enabled)


def _kept(ws: Tensor) -> Tensor:
    """The workspace the autograd context keeps for the backward."""
    return ws if _REUSE_FWD_WORKSPACE else ws.new_empty(0)


def _bwd_impl(do, q, k, v, o, lse, freqs, bias, mask, causal, softmax_scale, need_dfreqs, need_dbias,
              fwd_ws=None):
    q, k, v, o, do = (_unit_feature(t) for t in (q, k, v, o, do))
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    if not lse.is_contiguous():
        lse = lse.contiguous()
    _check_views(q, k, v, mask, lse)
    if o.shape != q.shape or do.shape != q.shape:
        raise ValueError(f"o {tuple(o.shape)} and do {tuple(do.shape)} must match q {tuple(q.shape)}")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    # the library clears dfreqs / dbias itself (POPE_FLAG_ZERO_GRADS) before accumulating, over the
    # key positions n < Nk it addresses; rows of a longer freqs table get no gradient, so such a
    # table's gradient starts from zeros
    long_freqs = need_dfreqs and freqs.shape[-2] > k.shape[2]
    alloc_df = torch.zeros if long_freqs else torch.empty
    dfreqs = alloc_df(freqs.shape, device=q.device, dtype=torch.float32) if need_dfreqs else q.new_empty(0, dtype=torch.float32)
    dbias = torch.empty(bias.shape, device=q.device, dtype=torch.float32) if need_dbias else q.new_empty(0, dtype=torch.float32)
    deterministic = _lib.deterministic_flag()
    key = ("bwd", deterministic, q.shape, q.stride(), k.shape, k.stride(), v.shape, v.stride(), o.stride(), do.stride(),
           dq.stride(), dk.stride(), dv.stride(), q.dtype, k.dtype, v.dtype, o.dtype, causal, softmax_scale,
           _opt_key(freqs), _opt_key(bias), _opt_key(mask), need_dfreqs, need_dbias)

    def build():
        _check_dtypes(q, k, v, o)
        _check_pope_shapes(q, k, freqs, bias)
        d = _desc(q, k, freqs, bias, causal, softmax_scale)
        d.q_s[:], d.k_s[:], d.v_s[:], d.o_s[:] = (_lib.strides3(t) for t in (q, k, v, o))
        d.do_s[:] = _lib.strides3(do)
        d.dq_s[:], d.dk_s[:], d.dv_s[:] = _lib.strides3(dq), _lib.strides3(dk), _lib.strides3(dv)
        if need_dfreqs:
            d.df_s[:] = _freqs_strides(dfreqs)
        if exists(mask):
            d.mask_sb = mask.stride(0)
        # torch.use_deterministic_algorithms(True): dfreqs / dbias summed in a fixed order
        d.flags = _lib.FLAG_ZERO_GRADS | deterministic
        # the same descriptor with PREPARED set, for calls that bring the forward's workspace
        dp = _lib.PopeDesc.from_buffer_copy(d)
        dp.flags |= _lib.FLAG_PREPARED
        return d, dp, _lib.workspace_bytes(_lib.OP_FLASH_BWD, d)

    d, dprep, need = _plan(key, build)
    global _LAST_BWD_PREPARED
    _LAST_BWD_PREPARED = exists(fwd_ws) and fwd_ws.numel() == need
    if _LAST_BWD_PREPARED:
        ws, d = fwd_ws, dprep
    else:
        ws = torch.empty(need, dtype=torch.uint8, device=q.device)
    st = _lib.lib().pope_flash_bwd(
        ctypes.byref(d), do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
        _data(freqs), _data(bias), _data(mask), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
        dfreqs.data_ptr() if need_dfreqs else None, dbias.data_ptr() if need_dbias else None,
        ws.data_ptr(), need, _stream(q))
    _lib.check(st, "flash backward")
    return dq, dk, dv, dfreqs, dbias


# ----------------------------------------------------------------------------- ops

@torch.library.custom_op("pope_amd::flash_fwd", mutates_args=(), device_types="cuda")
def flash_fwd_op(q: Tensor, k: Tensor, v: Tensor, freqs: Optional[Tensor], bias: Optional[Tensor],
                 mask: Optional[Tensor], causal: bool, softmax_scale: float) -> tuple[Tensor, Tensor, Tensor]:
    """q (B,Hq,Nq,D), k/v (B,Hk,Nk,D) bf16/fp16 views -> o like q, lse (B,Hq,Nq) fp32 and the
    workspace holding the forward's preparation (expanded K/Q rows, phase tables), which the
    backward reuses; empty when the decode kernel ran."""
    return _fwd_impl(q, k, v, freqs, bias, mask, causal, softmax_scale)


@flash_fwd_op.register_fake
def _(q, k, v, freqs, bias, mask, causal, softmax_scale):
    if _decode_eligible(q, k, v, freqs, causal):
        n = 0   # the decode kernel keeps nothing for the backward
    else:
        n = _fwd_ws_bytes(_desc(q, k, freqs, bias, causal, softmax_scale), _lib.deterministic_flag())
    return torch.empty_like(q), q.new_empty(q.shape[:3], dtype=torch.float32), q.new_empty(n, dtype=torch.uint8)


@torch.library.custom_op("pope_amd::flash_bwd", mutates_args=(), device_types="cuda")
def flash_bwd_op(do: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor,
                 freqs: Optional[Tensor], bias: Optional[Tensor], mask: Optional[Tensor], causal: bool,
                 softmax_scale: float, need_dfreqs: bool, need_dbias: bool, fwd_ws: Optional[Tensor] = None
                 ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients of flash_fwd.  ``fwd_ws`` is the workspace flash_fwd returned for the same
    inputs (reused as is); without it the preparation is recomputed."""
    return _bwd_impl(do, q, k, v, o, lse, freqs, bias, mask, causal, softmax_scale, need_dfreqs, need_dbias,
                     fwd_ws)


@flash_bwd_op.register_fake
def _(do, q, k, v, o, lse, freqs, bias, mask, causal, softmax_scale, need_dfreqs, need_dbias, fwd_ws=None):
    df = freqs.new_empty(freqs.shape, dtype=torch.float32) if need_dfreqs else q.new_empty(0, dtype=torch.float32)
    db = bias.new_empty(bias.shape, dtype=torch.float32) if need_dbias else q.new_empty(0, dtype=torch.float32)
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), df, db


def _fwd_setup(ctx, inputs, output):
    q, k, v, freqs, bias, mask, causal, scale = inputs
    o, lse, ws = output
    ctx.save_for_backward(q, k, v, freqs, bias, mask, o, lse, _kept(ws))
    ctx.causal, ctx.scale = causal, scale


def _fwd_backward(ctx, do, dlse, dws):
    q, k, v, freqs, bias, mask, o, lse, ws = ctx.saved_tensors
    need_df = bool(ctx.needs_input_grad[3]) and exists(freqs)
    need_db = bool(ctx.needs_input_grad[4]) and exists(bias)
    dq, dk, dv, df, db = flash_bwd_op(do, q, k, v, o, lse, freqs, bias, mask, ctx.causal, ctx.scale,
                                      need_df, need_db, ws)
    return (dq, dk, dv, df if need_df else None, db if need_db else None, None, None, None)


flash_fwd_op.register_autograd(_fwd_backward, setup_context=_fwd_setup)


class _FlashAttnEager(torch.autograd.Function):
    """The same forward / backward as the registered ops, called without the custom-op
    dispatch layers (about 20-30 us of host time per call).  Used outside torch.compile
    tracing; under tracing the ops above are used so the graph records them."""

    @staticmethod
    def forward(ctx, q, k, v, freqs, bias, mask, causal, scale):
        o, lse, ws = _fwd_impl(q, k, v, freqs, bias, mask, causal, scale)
        ctx.save_for_backward(q, k, v, freqs, bias, mask, o, lse, _kept(ws))
        ctx.causal, ctx.scale = causal, scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, freqs, bias, mask, o, lse, ws = ctx.saved_tensors
        need_df = bool(ctx.needs_input_grad[3]) and exists(freqs)
        need_db = bool(ctx.needs_input_grad[4]) and exists(bias)
        dq, dk, dv, df, db = _bwd_impl(do, q, k, v, o, lse, freqs, bias, mask, ctx.causal, ctx.scale,
                                       need_df, need_db, ws)
        return dq, dk, dv, df if need_df else None, db if need_db else None, None, None, None


def _flash(q, k, v, freqs, bias, mask, causal, scale) -> Tensor:
    if torch.compiler.is_compiling():
        return flash_fwd_op(q, k, v, freqs, bias, mask, causal, scale)[0]
    return _FlashAttnEager.apply(q, k, v, freqs, bias, mask, causal, scale)


# ------------------------------------------------------------ head-first entry point

def flash_attn_head_first(q: Tensor, k: Tensor, v: Tensor, freqs: Optional[Tensor] = None,
                          pope_bias: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                          causal: bool = False, softmax_scale: Optional[float] = None) -> Tensor:
    """Differentiable PoPE flash attention on (B, H, N, D) views -> o (B, Hq, Nq, D)."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("pope_amd flash attention runs on GPU tensors only")
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    freqs, pope_bias = _prep_pope(freqs, pope_bias)
    mask = _prep_mask(mask, q.shape[0])
    out_dtype = q.dtype
    if q.dtype not in _MFMA_DTYPES:
        # fp32 inputs: fp16 operands keep 10 significant bits, as the TF32 products of the
        # reference's fp32 path do (triton_pope_flash_attn.py:80), but not TF32's exponent range
        _check_fp16_range(q, k, v)
        q, k, v = q.to(torch.float16), k.to(torch.float16), v.to(torch.float16)
    if k.dtype != q.dtype:
        k = k.to(q.dtype)
    if v.dtype != q.dtype:
        v = v.to(q.dtype)
    # head / rotate dims that are not multiples of 8: padded on the device (pope_amd._pad)
    plan = pad_plan(q.shape[-1], freqs.shape[-1] if exists(freqs) else 0)
    if plan is not None:
        q, k, v = pad_qk(q, plan), pad_qk(k, plan), pad_last(v, plan.Dp)
        freqs, pope_bias = pad_last(freqs, plan.R8), pad_last(pope_bias, plan.R8)
    o = _flash(q, k, v, freqs, pope_bias, mask, causal, float(scale))
    if plan is not None:
        o = o[..., :plan.D]
    return o.to(out_dtype) if o.dtype != out_dtype else o


# ------------------------------------------------- reference-named (b, n, h, d) API

def flash_attn_forward(q, k, v, freqs=None, pope_bias=None, mask=None, causal=False, softmax_scale=None):
    """(B, N, H, D) tensors -> (o, lse); triton_pope_flash_attn.py:222-271."""
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    freqs, pope_bias = _prep_pope(freqs, pope_bias)
    mask = _prep_mask(mask, q.shape[0])
    qh, kh, vh = (t.transpose(1, 2) for t in (q, k, v))
    if exists(freqs) and freqs.ndim == 4:
        freqs = freqs.transpose(1, 2)   # (B, N, H, R) -> (B, H, N, R) view
    plan = pad_plan(q.shape[-1], freqs.shape[-1] if exists(freqs) else 0)
    if plan is not None:
        qh, kh, vh = pad_qk(qh, plan), pad_qk(kh, plan), pad_last(vh, plan.Dp)
        freqs, pope_bias = pad_last(freqs, plan.R8), pad_last(pope_bias, plan.R8)
    o, lse, _ = flash_fwd_op(qh, kh, vh, freqs, pope_bias, mask, causal, float(scale))
    if plan is not None:
        o = o[..., :plan.D]
    return o.transpose(1, 2), lse


def flash_attn_backward(do, q, k, v, o, lse, dq, dk, dv, dfreqs=None, dpope_bias=None, freqs=None,
                        pope_bias=None, mask=None, causal=False, softmax_scale=None):
    """Gradients into caller tensors, (B, N, H, D) layout; triton_pope_flash_attn.py:273-335.

    The same write semantics as the reference launcher: dq, dfreqs and dpope_bias are added to
    (its kernel accumulates them with atomics, :207-210,215, into buffers the caller zeroes,
    :358-359), dk and dv are overwritten (:217-218)."""
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    freqs, pope_bias = _prep_pope(freqs, pope_bias)
    mask = _prep_mask(mask, q.shape[0])
    tr = lambda t: t.transpose(1, 2)
    f = freqs.transpose(1, 2) if exists(freqs) and freqs.ndim == 4 else freqs
    tq, tk, tv, to, tdo = tr(q), tr(k), tr(v), tr(o), tr(do)
    plan = pad_plan(q.shape[-1], freqs.shape[-1] if exists(freqs) else 0)
    if plan is not None:
        tq, tk = pad_qk(tq, plan), pad_qk(tk, plan)
        tv, to, tdo = pad_last(tv, plan.Dp), pad_last(to, plan.Dp), pad_last(tdo, plan.Dp)
        f, pope_bias = pad_last(f, plan.R8), pad_last(pope_bias, plan.R8)
    gq, gk, gv, gf, gb = flash_bwd_op(tdo, tq, tk, tv, to, lse, f, pope_bias, mask, causal,
                                      float(scale), exists(dfreqs), exists(dpope_bias))
    if plan is not None:
        gq, gk, gv = unpad_qk(gq, plan), unpad_qk(gk, plan), gv[..., :plan.D]
        gf = gf[..., :plan.R] if exists(dfreqs) else gf
        gb = gb[..., :plan.R] if exists(dpope_bias) else gb
    dq.add_(tr(gq))
    dk.copy_(tr(gk))
    dv.copy_(tr(gv))
    if exists(dfreqs):
        dfreqs.add_(gf.transpose(1, 2) if gf.ndim == 4 else gf)
    if exists(dpope_bias):
        dpope_bias.add_(gb.reshape(dpope_bias.shape))


class FlashAttnFunction:
    """Name-compatible stand-in for the reference's autograd Function
    (triton_pope_flash_attn.py:337-362); differentiation comes from the
    registered autograd of ``pope_amd::flash_fwd``."""

    @staticmethod
    def apply(q, k, v, freqs=None, pope_bias=None, mask=None, causal=False, softmax_scale=None):
        o, _ = flash_attn_forward(q, k, v, freqs, pope_bias, mask, causal, softmax_scale)
        return o


def flash_attn(q, k, v, freqs=None, pope_bias=None, mask=None, causal=False, softmax_scale=None):
    """(B, N, H, D) flash attention with PoPE; triton_pope_flash_attn.py:364-373 (no copies)."""
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    if exists(freqs) and freqs.ndim == 4:
        freqs = freqs.transpose(1, 2)
    o = flash_attn_head_first(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), freqs, pope_bias,
                              mask, causal, scale)
    return o.transpose(1, 2)
