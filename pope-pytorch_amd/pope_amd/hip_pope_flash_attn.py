"""Flash attention with PoPE on the HIP kernels of libpope_hip.so.

Operator mirror of the reference's ``PoPE_pytorch/triton_pope_flash_attn.py``:
``flash_attn_forward`` (:222-271), ``flash_attn_backward`` (:273-335),
``FlashAttnFunction`` (:337-362) and ``flash_attn`` (:364-373) keep their names,
arguments, (batch, seq, heads, dim) layout and return values.  Underneath, two
``torch.library`` custom ops carry the work:

  pope_amd::flash_fwd(q, k, v, freqs?, bias?, mask?, causal, scale) -> (o, lse)
  pope_amd::flash_bwd(do, q, k, v, o, lse, freqs?, bias?, mask?, causal, scale,
                      need_dfreqs, need_dbias) -> (dq, dk, dv, dfreqs, dbias)

with ``flash_fwd`` differentiable through ``register_autograd``.  The ops take
head-first logical views (B, H, N, D) with any batch/head/seq strides and a unit
feature stride, so the (b n h d) <-> (b h n d) permutes of the reference cost no
copies.  Query head h reads kv head h % Hk (the reference's torch-path GQA
mapping, attention.py:118-120; the reference's fused kernel has no GQA).

Differences from the reference kernels, by design:
  * dq is accumulated in fp32 (the reference adds bf16 atomics, :215,358);
  * the backward skips key/query tiles past the causal diagonal (:167 visits all);
  * out-of-range keys are always masked (:152-199 leaves them in when the call is
    non-causal, unmasked and Nk % 32 != 0);
  * fp32 inputs run the bf16 MFMA kernels on bf16-rounded q, k, v (the reference
    runs tl.dot at TF32 for fp32, which is likewise a reduced-precision product).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import _lib

_MFMA_DTYPES = (torch.bfloat16, torch.float16)


def exists(v):
    return v is not None


def _freqs_strides(freqs: Tensor, head_first: bool = True) -> tuple:
    """(b, h, n) element strides of a freqs table (r stride must be 1).

    2-D (N, R): shared; 3-D (B, N, R): per batch; 4-D: (B, H, N, R) head-first
    or (B, N, H, R) when the caller works in (batch, seq, heads) layout
    (triton_pope_flash_attn.py:237-245)."""
    s = freqs.stride()
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
    if freqs.stride(-1) != 1:
        freqs = freqs.contiguous()
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


# ----------------------------------------------------------------------------- ops

@torch.library.custom_op("pope_amd::flash_fwd", mutates_args=(), device_types="cuda")
def flash_fwd_op(q: Tensor, k: Tensor, v: Tensor, freqs: Optional[Tensor], bias: Optional[Tensor],
                 mask: Optional[Tensor], causal: bool, softmax_scale: float) -> tuple[Tensor, Tensor, Tensor]:
    """q (B,Hq,Nq,D), k/v (B,Hk,Nk,D) bf16/fp16 views -> o like q, lse (B,Hq,Nq) fp32 and the
    workspace holding the forward's preparation (expanded K/Q rows, phase tables), which the
    backward reuses; empty when the decode kernel ran."""
    L = _lib.lib()
    q, k, v = _unit_feature(q), _unit_feature(k), _unit_feature(v)
    d = _desc(q, k, freqs, bias, causal, softmax_scale)
    d.q_s[:], d.k_s[:], d.v_s[:] = _lib.strides3(q), _lib.strides3(k), _lib.strides3(v)
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    d.o_s[:] = _lib.strides3(o)
    if exists(mask):
        d.mask_sb = mask.stride(0)
    args = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(freqs), _lib.ptr(bias), _lib.ptr(mask),
            _lib.ptr(o), _lib.ptr(lse))
    stream = _lib.stream_ptr(q.device)
    # one non-causal query row against a long cache: the split-K decode kernel
    if q.shape[2] == 1 and not causal and k.shape[2] >= 1024:
        dws = _lib.workspace(_lib.OP_FLASH_DECODE, d, q.device)
        st = L.pope_flash_decode(ctypes.byref(d), *args, _lib.ptr(dws), 0 if dws is None else dws.numel(), stream)
        if st == 0:
            return o, lse, q.new_empty(0, dtype=torch.uint8)
        if st != 2:   # 2: the decode kernel does not cover this shape -> general forward
            _lib.check(st, "flash decode")
    ws = _lib.workspace(_lib.OP_FLASH_FWD, d, q.device)
    st = L.pope_flash_fwd(ctypes.byref(d), *args, _lib.ptr(ws), ws.numel(), stream)
    _lib.check(st, "flash forward")
    return o, lse, ws


@flash_fwd_op.register_fake
def _(q, k, v, freqs, bias, mask, causal, softmax_scale):
    d = _desc(q, k, freqs, bias, causal, softmax_scale)
    n = _lib.workspace_bytes(_lib.OP_FLASH_FWD, d)
    return torch.empty_like(q), q.new_empty(q.shape[:3], dtype=torch.float32), q.new_empty(n, dtype=torch.uint8)


@torch.library.custom_op("pope_amd::flash_bwd", mutates_args=(), device_types="cuda")
def flash_bwd_op(do: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor,
                 freqs: Optional[Tensor], bias: Optional[Tensor], mask: Optional[Tensor], causal: bool,
                 softmax_scale: float, need_dfreqs: bool, need_dbias: bool, fwd_ws: Optional[Tensor] = None
                 ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients of flash_fwd.  ``fwd_ws`` is the workspace flash_fwd returned for the same
    inputs (reused as is); without it the preparation is recomputed."""
    L = _lib.lib()
    q, k, v, o, do = (_unit_feature(t) for t in (q, k, v, o, do))
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    d = _desc(q, k, freqs, bias, causal, softmax_scale)
    d.q_s[:], d.k_s[:], d.v_s[:], d.o_s[:] = (_lib.strides3(t) for t in (q, k, v, o))
    d.do_s[:] = _lib.strides3(do)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    d.dq_s[:], d.dk_s[:], d.dv_s[:] = _lib.strides3(dq), _lib.strides3(dk), _lib.strides3(dv)
    # the library clears dfreqs / dbias itself (POPE_FLAG_ZERO_GRADS) before accumulating
    dfreqs = torch.empty(freqs.shape, device=q.device, dtype=torch.float32) if need_dfreqs else q.new_empty(0, dtype=torch.float32)
    dbias = torch.empty(bias.shape, device=q.device, dtype=torch.float32) if need_dbias else q.new_empty(0, dtype=torch.float32)
    if need_dfreqs:
        d.df_s[:] = _freqs_strides(dfreqs)
    if exists(mask):
        d.mask_sb = mask.stride(0)
    d.flags = _lib.FLAG_ZERO_GRADS
    need = _lib.workspace_bytes(_lib.OP_FLASH_BWD, d)
    if exists(fwd_ws) and fwd_ws.numel() == need:
        ws = fwd_ws
        d.flags |= _lib.FLAG_PREPARED
    else:
        ws = torch.empty(need, dtype=torch.uint8, device=q.device)
    st = L.pope_flash_bwd(ctypes.byref(d), _lib.ptr(do), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o),
                          _lib.ptr(lse), _lib.ptr(freqs), _lib.ptr(bias), _lib.ptr(mask), _lib.ptr(dq),
                          _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dfreqs) if need_dfreqs else None,
                          _lib.ptr(dbias) if need_dbias else None, _lib.ptr(ws), ws.numel(),
                          _lib.stream_ptr(q.device))
    _lib.check(st, "flash backward")
    return dq, dk, dv, dfreqs, dbias


@flash_bwd_op.register_fake
def _(do, q, k, v, o, lse, freqs, bias, mask, causal, softmax_scale, need_dfreqs, need_dbias, fwd_ws=None):
    df = freqs.new_empty(freqs.shape, dtype=torch.float32) if need_dfreqs else q.new_empty(0, dtype=torch.float32)
    db = bias.new_empty(bias.shape, dtype=torch.float32) if need_dbias else q.new_empty(0, dtype=torch.float32)
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), df, db


def _fwd_setup(ctx, inputs, output):
    q, k, v, freqs, bias, mask, causal, scale = inputs
    o, lse, ws = output
    ctx.save_for_backward(q, k, v, freqs, bias, mask, o, lse, ws)
    ctx.causal, ctx.scale = causal, scale


def _fwd_backward(ctx, do, dlse, dws):
    q, k, v, freqs, bias, mask, o, lse, ws = ctx.saved_tensors
    need_df = bool(ctx.needs_input_grad[3]) and exists(freqs)
    need_db = bool(ctx.needs_input_grad[4]) and exists(bias)
    dq, dk, dv, df, db = flash_bwd_op(do, q, k, v, o, lse, freqs, bias, mask, ctx.causal, ctx.scale,
                                      need_df, need_db, ws)
    return (dq, dk, dv, df if need_df else None, db if need_db else None, None, None, None)


flash_fwd_op.register_autograd(_fwd_backward, setup_context=_fwd_setup)


# ------------------------------------------------------------ head-first entry point

def flash_attn_head_first(q: Tensor, k: Tensor, v: Tensor, freqs: Optional[Tensor] = None,
                          pope_bias: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                          causal: bool = False, softmax_scale: Optional[float] = None) -> Tensor:
    """Differentiable PoPE flash attention on (B, H, N, D) views -> o (B, Hq, Nq, D)."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("pope_amd flash attention runs on GPU tensors only")
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    freqs, pope_bias = _prep_pope(freqs, pope_bias)
    _check_pope_shapes(q, k, freqs, pope_bias)
    mask = _prep_mask(mask, q.shape[0])
    out_dtype = q.dtype
    if q.dtype not in _MFMA_DTYPES:
        q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    if k.dtype != q.dtype:
        k = k.to(q.dtype)
    if v.dtype != q.dtype:
        v = v.to(q.dtype)
    o, _, _ = flash_fwd_op(q, k, v, freqs, pope_bias, mask, causal, float(scale))
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
    o, lse, _ = flash_fwd_op(qh, kh, vh, freqs, pope_bias, mask, causal, float(scale))
    return o.transpose(1, 2), lse


def flash_attn_backward(do, q, k, v, o, lse, dq, dk, dv, dfreqs=None, dpope_bias=None, freqs=None,
                        pope_bias=None, mask=None, causal=False, softmax_scale=None):
    """Writes grads into caller tensors, (B, N, H, D) layout; triton_pope_flash_attn.py:273-335."""
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    freqs, pope_bias = _prep_pope(freqs, pope_bias)
    mask = _prep_mask(mask, q.shape[0])
    tr = lambda t: t.transpose(1, 2)
    f = freqs.transpose(1, 2) if exists(freqs) and freqs.ndim == 4 else freqs
    gq, gk, gv, gf, gb = flash_bwd_op(tr(do), tr(q), tr(k), tr(v), tr(o), lse, f, pope_bias, mask, causal,
                                      float(scale), exists(dfreqs), exists(dpope_bias))
    dq.copy_(tr(gq))
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
