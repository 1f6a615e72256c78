"""Materialising polar transform on the HIP kernels of libpope_hip.so.

The device form of the reference's ``apply_pope_to_qk`` (pope.py:30-86) with its
default softplus magnitude: ``pope_amd::polar_fwd`` writes q_hat / k_hat
(fp32, last dim D + R, interleaved (a cos, a sin) per rotated dim, then the raw
pass-through dims) and ``pope_amd::polar_bwd`` is its autograd backward (dq, dk
in the input dtype; dfreqs / dbias when they require grad).  With ``complex=True``
the kernels write the complex64 layout of ``return_complex=True`` (pope.py:49-51,
66-67,74-75: D (re, im) pairs per row, pass-through dims as (x, 0)), returned as
``torch.view_as_complex`` views, through which autograd hands the kernels the
gradient pairs.
``pope.apply_pope_to_qk`` routes CUDA tensors here when the call fits the
kernels (4-D q / k, fp32 freqs and bias, default magnitude; fp32 q / k for the
complex output) and keeps the torch ops otherwise.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib
from ._pad import pad_last, pad_plan, pad_qk
from .hip_pope_flash_attn import _freqs_strides


def _desc(q: Tensor, k: Tensor, freqs: Tensor, bias: Tensor, complex_out: bool) -> _lib.PopeDesc:
    d = _lib.PopeDesc()
    d.B, d.Hq, d.Nq, d.D = q.shape
    d.Hk, d.Nk = k.shape[1], k.shape[2]
    d.R = freqs.shape[-1]
    d.dtype = _lib.dtype_code(q.dtype)
    d.flags = _lib.FLAG_COMPLEX if complex_out else 0
    d.q_s[:], d.k_s[:] = _lib.strides3(q), _lib.strides3(k)
    d.f_s[:] = _freqs_strides(freqs)
    d.bias_sh = bias.stride(0) if bias.shape[0] > 1 else 0
    return d


def _rows4(t: Tensor) -> Tensor:
    """Unit feature stride, other strides multiples of 4 elements, 16-byte aligned start."""
    if t.stride(-1) != 1 or any(s % 4 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
        if t.data_ptr() % 16:
            t = t.clone()
    return t


def _width(D: int, R: int, complex_out: bool) -> int:
    """fp32 columns per output row: D + R, or D (re, im) pairs."""
    return 2 * D if complex_out else D + R


@torch.library.custom_op("pope_amd::polar_fwd", mutates_args=(), device_types="cuda")
def polar_fwd_op(q: Tensor, k: Tensor, freqs: Tensor, bias: Tensor, complex_out: bool = False) -> tuple[Tensor, Tensor]:
    q, k = _rows4(q), _rows4(k)
    d = _desc(q, k, freqs, bias, complex_out)
    E = _width(q.shape[-1], freqs.shape[-1], complex_out)
    qh = torch.empty(*q.shape[:3], E, device=q.device, dtype=torch.float32)
    kh = torch.empty(*k.shape[:3], E, device=q.device, dtype=torch.float32)
    st = _lib.lib().pope_polar_fwd(ctypes.byref(d), _lib.ptr(q), _lib.ptr(k), _lib.ptr(freqs), _lib.ptr(bias),
                                   _lib.ptr(qh), _lib.ptr(kh), _lib.stream_ptr(q.device))
    _lib.check(st, "polar transform")
    return qh, kh


@polar_fwd_op.register_fake
def _(q, k, freqs, bias, complex_out=False):
    E = _width(q.shape[-1], freqs.shape[-1], complex_out)
    return (q.new_empty((*q.shape[:3], E), dtype=torch.float32), k.new_empty((*k.shape[:3], E), dtype=torch.float32))


@torch.library.custom_op("pope_amd::polar_bwd", mutates_args=(), device_types="cuda")
def polar_bwd_op(gq: Tensor, gk: Tensor, q: Tensor, k: Tensor, freqs: Tensor, bias: Tensor, need_dfreqs: bool,
                 need_dbias: bool, complex_out: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    q, k = _rows4(q), _rows4(k)
    gq, gk = gq.float().contiguous(), gk.float().contiguous()
    d = _desc(q, k, freqs, bias, complex_out)
    d.flags |= _lib.deterministic_flag()   # torch.use_deterministic_algorithms(True): no fp32 atomics
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    d.dq_s[:], d.dk_s[:] = _lib.strides3(dq), _lib.strides3(dk)
    empty = q.new_empty(0, dtype=torch.float32)
    dfreqs = torch.zeros(freqs.shape, device=q.device, dtype=torch.float32) if need_dfreqs else empty
    dbias = torch.zeros(bias.shape, device=q.device, dtype=torch.float32) if need_dbias else empty
    if need_dfreqs:
        d.df_s[:] = _freqs_strides(dfreqs)
    ws = _lib.workspace(_lib.OP_POLAR_BWD, d, q.device)
    st = _lib.lib().pope_polar_bwd(ctypes.byref(d), _lib.ptr(gq), _lib.ptr(gk), _lib.ptr(q), _lib.ptr(k),
                                   _lib.ptr(freqs), _lib.ptr(bias), _lib.ptr(dq), _lib.ptr(dk),
                                   _lib.ptr(dfreqs) if need_dfreqs else None,
                                   _lib.ptr(dbias) if need_dbias else None, _lib.ptr(ws),
                                   0 if ws is None else ws.numel(), _lib.stream_ptr(q.device))
    _lib.check(st, "polar transform backward")
    return dq, dk, dfreqs, dbias


@polar_bwd_op.register_fake
def _(gq, gk, q, k, freqs, bias, need_dfreqs, need_dbias, complex_out=False):
    df = freqs.new_empty(freqs.shape, dtype=torch.float32) if need_dfreqs else q.new_empty(0, dtype=torch.float32)
    db = bias.new_empty(bias.shape, dtype=torch.float32) if need_dbias else q.new_empty(0, dtype=torch.float32)
    return torch.empty_like(q), torch.empty_like(k), df, db


def _setup(ctx, inputs, output):
    q, k, freqs, bias, complex_out = inputs
    ctx.save_for_backward(q, k, freqs, bias)
    ctx.complex_out = complex_out


def _backward(ctx, gq, gk):
    q, k, freqs, bias = ctx.saved_tensors
    R = freqs.shape[-1]
    E = _width(q.shape[-1], R, ctx.complex_out)
    need_df = bool(ctx.needs_input_grad[2]) and R > 0
    need_db = bool(ctx.needs_input_grad[3]) and R > 0
    if gq is None:
        gq = torch.zeros(*q.shape[:3], E, device=q.device)
    if gk is None:
        gk = torch.zeros(*k.shape[:3], E, device=k.device)
    dq, dk, df, db = polar_bwd_op(gq, gk, q, k, freqs, bias, need_df, need_db, ctx.complex_out)
    return dq, dk, df.to(freqs.dtype) if need_df else None, db.to(bias.dtype) if need_db else None, None


polar_fwd_op.register_autograd(_backward, setup_context=_setup)


def fits(q: Tensor, k: Tensor, freqs: Tensor, bias: Tensor, to_magnitude, return_complex: bool) -> bool:
    """Whether apply_pope_to_qk(pos, q, k, ...) can run on the kernels."""
    if to_magnitude is not F.softplus:
        return False
    if not (q.is_cuda and k.is_cuda and freqs.is_cuda and bias.is_cuda):
        return False
    if q.ndim != 4 or k.ndim != 4 or q.dtype != k.dtype or q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return False
    if return_complex and q.dtype != torch.float32:
        return False   # torch.polar takes the softplus magnitude in q's dtype: fp32 only (pope.py:67)
    if freqs.dtype != torch.float32 or bias.dtype != torch.float32 or bias.ndim != 2 or freqs.stride(-1) != 1:
        return False
    if freqs.ndim not in (2, 3) or (freqs.ndim == 3 and freqs.shape[0] != q.shape[0]):
        return False
    B, Hq, Nq, D = q.shape
    R = freqs.shape[-1]
    plan = pad_plan(D, R)   # head / rotate dims not multiples of 8: padded in polar()
    if k.shape[0] != B or k.shape[-1] != D or (plan.Dp if plan else D) > 512 or R > D or Nq > k.shape[2] or R == 0:
        return False
    if bias.shape[-1] != R or bias.shape[0] not in (1, k.shape[1]) or bias.stride(-1) != 1:
        return False
    return freqs.shape[-2] == k.shape[2]


def polar(q: Tensor, k: Tensor, freqs: Tensor, bias: Tensor, return_complex: bool = False) -> tuple[Tensor, Tensor]:
    D, R = q.shape[-1], freqs.shape[-1]
    plan = pad_plan(D, R)
    if plan is not None:
        # rows padded on the device (pope_amd._pad); the padded dims' output columns are dropped
        q, k = pad_qk(q, plan), pad_qk(k, plan)
        freqs, bias = pad_last(freqs, plan.R8), pad_last(bias, plan.R8)
    qh, kh = polar_fwd_op(q, k, freqs, bias, return_complex)
    if return_complex:
        W = q.shape[-1]
        qh = torch.view_as_complex(qh.view(*qh.shape[:-1], W, 2))
        kh = torch.view_as_complex(kh.view(*kh.shape[:-1], W, 2))
        if plan is not None:   # complex dims: R rotated, then D - R pass-through
            keep = lambda t: torch.cat([t[..., :R], t[..., plan.R8:plan.R8 + D - R]], -1)
            qh, kh = keep(qh), keep(kh)
    elif plan is not None:     # real columns: 2 R interleaved (cos, sin) pairs, then D - R pass-through
        keep = lambda t: torch.cat([t[..., :2 * R], t[..., 2 * plan.R8:2 * plan.R8 + D - R]], -1)
        qh, kh = keep(qh), keep(kh)
    return qh, kh
