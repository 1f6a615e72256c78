"""Fused PoPE attention similarity on the HIP kernels of libpope_hip.so.

Operator mirror of the reference's ``PoPE_pytorch/triton_pope.py``:
``PoPESimilarityFunction`` (:258-362) and ``triton_compute_qk_similarity``
(:364-372, here ``hip_compute_qk_similarity``) keep their arguments and return
values.  The work runs in two ``torch.library`` custom ops:

  pope_amd::sim_fwd(q, k, freqs, bias, split) -> sim
  pope_amd::sim_bwd(dsim, q, k, freqs, bias, need_dfreqs, need_dbias, split)
                                      -> (dq, dk, dfreqs, dbias)

``sim_fwd`` is differentiable through ``register_autograd``.  Query head h reads
kv head h % Hk and bias row h % Hk, which is what the reference's repeat of k and
bias (:368-370) amounts to, without materialising the repeat.

``allow_tf32`` selects the product arithmetic, as it does in the reference
(triton_pope.py:63,145,224): ``True`` (the default) runs the products on bf16
MFMA with every fp32 operand split into hi + lo bf16 halves (``split=True``:
three products per pair, 16 significant operand bits, fp32 accumulation; the
reference's TF32 keeps 10), ``False`` runs true fp32 MFMA (the reference's tests
pass ``allow_tf32=False`` for their parity checks, test_triton.py:300,335,359).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from ._pad import pad_last, pad_plan, pad_qk
from .hip_pope_flash_attn import _freqs_strides


def exists(v):
    return v is not None


def divisible_by(num, den):
    return (num % den) == 0


def _desc(q, k, freqs, bias, split=False) -> _lib.PopeDesc:
    B, Hq, Nq, D = q.shape
    d = _lib.PopeDesc()
    d.flags = _lib.FLAG_SPLIT_BF16 if split else 0
    d.B, d.Hq, d.Hk, d.Nq, d.Nk, d.D = B, Hq, k.shape[1], Nq, k.shape[2], D
    d.R = freqs.shape[-1]
    d.dtype = _lib.POPE_F32
    d.q_s[:], d.k_s[:] = _lib.strides3(q), _lib.strides3(k)
    d.f_s[:] = _freqs_strides(freqs)
    d.bias_sh = bias.stride(0) if bias.shape[0] > 1 else 0
    return d


def _aligned(t: Tensor) -> Tensor:
    """fp32 views with unit feature stride and 16-byte aligned rows (the kernels use float4 loads)."""
    if t.stride(-1) != 1 or any(s % 4 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
        if t.data_ptr() % 16:
            t = t.clone()
    return t


@torch.library.custom_op("pope_amd::sim_fwd", mutates_args=(), device_types="cuda")
def sim_fwd_op(q: Tensor, k: Tensor, freqs: Tensor, bias: Tensor, split: bool = False) -> Tensor:
    """q (B,Hq,Nq,D), k (B,Hk,Nk,D) fp32; freqs (..,N,R) fp32; bias (1|Hk,R) -> sim (B,Hq,Nq,Nk) fp32.
    split: products on split-bf16 MFMA instead of fp32 MFMA."""
    L = _lib.lib()
    q, k = _aligned(q), _aligned(k)
    d = _desc(q, k, freqs, bias, split)
    sim = torch.empty(q.shape[0], q.shape[1], q.shape[2], k.shape[2], device=q.device, dtype=torch.float32)
    d.sim_s[:] = _lib.strides3(sim)
    ws = _lib.workspace(_lib.OP_SIM_FWD, d, q.device)
    st = L.pope_sim_fwd(ctypes.byref(d), _lib.ptr(q), _lib.ptr(k), _lib.ptr(freqs), _lib.ptr(bias), _lib.ptr(sim),
                        _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_ptr(q.device))
    _lib.check(st, "similarity forward")
    return sim


@sim_fwd_op.register_fake
def _(q, k, freqs, bias, split=False):
    return q.new_empty((q.shape[0], q.shape[1], q.shape[2], k.shape[2]), dtype=torch.float32)


@torch.library.custom_op("pope_amd::sim_bwd", mutates_args=(), device_types="cuda")
def sim_bwd_op(dsim: Tensor, q: Tensor, k: Tensor, freqs: Tensor, bias: Tensor, need_dfreqs: bool,
               need_dbias: bool, split: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    L = _lib.lib()
    q, k, dsim = _aligned(q), _aligned(k), _aligned(dsim.float())
    d = _desc(q, k, freqs, bias, split)
    d.flags |= _lib.deterministic_flag()   # torch.use_deterministic_algorithms(True): no fp32 atomics
    # the library clears dfreqs / dbias before accumulating into them, over the positions n < Nk
    # it addresses; rows of a longer freqs table get no gradient, so that gradient starts from zeros
    d.flags |= _lib.FLAG_ZERO_GRADS
    d.sim_s[:] = _lib.strides3(dsim)
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    d.dq_s[:], d.dk_s[:] = _lib.strides3(dq), _lib.strides3(dk)
    alloc_df = torch.zeros if freqs.shape[-2] > k.shape[2] else torch.empty
    dfreqs = alloc_df(freqs.shape, device=q.device, dtype=torch.float32) if need_dfreqs else q.new_empty(0, dtype=torch.float32)
    dbias = torch.empty(bias.shape, device=q.device, dtype=torch.float32) if need_dbias else q.new_empty(0, dtype=torch.float32)
    if need_dfreqs:
        d.df_s[:] = _freqs_strides(dfreqs)
    ws = _lib.workspace(_lib.OP_SIM_BWD, d, q.device)
    st = L.pope_sim_bwd(ctypes.byref(d), _lib.ptr(dsim), _lib.ptr(q), _lib.ptr(k), _lib.ptr(freqs), _lib.ptr(bias),
                        _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dfreqs) if need_dfreqs else None,
                        _lib.ptr(dbias) if need_dbias else None, _lib.ptr(ws), 0 if ws is None else ws.numel(),
                        _lib.stream_ptr(q.device))
    _lib.check(st, "similarity backward")
    return dq, dk, dfreqs, dbias


@sim_bwd_op.register_fake
def _(dsim, q, k, freqs, bias, need_dfreqs, need_dbias, split=False):
    df = freqs.new_empty(freqs.shape, dtype=torch.float32) if need_dfreqs else q.new_empty(0, dtype=torch.float32)
    db = bias.new_empty(bias.shape, dtype=torch.float32) if need_dbias else q.new_empty(0, dtype=torch.float32)
    return torch.empty_like(q), torch.empty_like(k), df, db


def _sim_setup(ctx, inputs, output):
    q, k, freqs, bias, split = inputs
    ctx.save_for_backward(q, k, freqs, bias)
    ctx.split = split


def _sim_backward(ctx, dsim):
    q, k, freqs, bias = ctx.saved_tensors
    need_df = bool(ctx.needs_input_grad[2]) and freqs.shape[-1] > 0
    need_db = bool(ctx.needs_input_grad[3]) and bias.shape[-1] > 0
    dq, dk, df, db = sim_bwd_op(dsim, q, k, freqs, bias, need_df, need_db, ctx.split)
    return dq, dk, df if need_df else None, db if need_db else None, None


sim_fwd_op.register_autograd(_sim_backward, setup_context=_sim_setup)


def _prep(q, k, freqs, bias):
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


class PoPESimilarityFunction:
    """Name-compatible stand-in for the reference's autograd Function
    (triton_pope.py:258-362): ``apply(q, k, freqs, bias, rotate_dim, allow_tf32)``."""

    @staticmethod
    def apply(q, k, freqs, bias, rotate_dim=None, allow_tf32=True):
        return hip_compute_qk_similarity(q, k, freqs, bias, rotate_dim, allow_tf32)


def hip_compute_qk_similarity(q, k, freqs, bias, rotate_dim=None, allow_tf32=True):
    """Unscaled PoPE similarity of (B, Hq, Nq, D) q and (B, Hk, Nk, D) k on the GPU
    (triton_pope.py:364-372).  Returns sim (B, Hq, Nq, Nk) in q's dtype."""
    assert divisible_by(q.shape[1], k.shape[1])
    if not (q.is_cuda and k.is_cuda):
        raise RuntimeError("pope_amd fused similarity runs on GPU tensors only")
    freqs, bias = _prep(q, k, freqs, bias)
    if rotate_dim is not None and rotate_dim != freqs.shape[-1]:
        raise ValueError(f"rotate_dim {rotate_dim} != freqs.shape[-1] {freqs.shape[-1]}")
    R = freqs.shape[-1]
    if R > q.shape[-1]:
        raise AssertionError(f"rotate dim {R} exceeds head dim {q.shape[-1]}")
    if R > 0 and (bias.shape[-1] != R or bias.shape[0] not in (1, k.shape[1])):
        raise ValueError(f"bias {tuple(bias.shape)} must be (1 or {k.shape[1]}, {R})")
    if freqs.shape[-2] < k.shape[2]:
        raise ValueError(f"freqs has {freqs.shape[-2]} positions, keys need {k.shape[2]}")
    out_dtype = q.dtype
    qf, kf = q.float(), k.float()
    # head / rotate dims that are not multiples of 8: padded on the device (pope_amd._pad)
    plan = pad_plan(q.shape[-1], R)
    if plan is not None:
        qf, kf = pad_qk(qf, plan), pad_qk(kf, plan)
        freqs, bias = pad_last(freqs, plan.R8), pad_last(bias, plan.R8)
    sim = sim_fwd_op(qf, kf, freqs, bias, bool(allow_tf32))
    return sim.to(out_dtype) if out_dtype != torch.float32 else sim
