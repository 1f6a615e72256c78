"""Head dims and rotate dims that are not multiples of 8.

The HIP kernels move rows in 16-byte chunks, so the C ABI takes a head dim D and a rotate dim R
that are multiples of 8.  The reference's kernels take any D and R (Triton blocks of
next_pow2(D) with a rotate mask, triton_pope.py:58-60, triton_pope_flash_attn.py:44,252).  The
Python entry points reach the same results by padding, on the device, before the kernels run:

  q, k   (.., D)  ->  (.., R8 + P8) = [x[:R] | PAD_LOGIT x (R8 - R) | x[R:] | 0 x (P8 - (D - R))]
  v, o, dO        ->  zeros appended up to R8 + P8
  freqs, bias     ->  zeros appended up to R8

with R8 = ceil8(R), P8 = ceil8(D - R).  A padded rotated dim has magnitude softplus(PAD_LOGIT),
which is exactly 0 in fp32 (e^-10000 underflows), so it adds nothing to any score and its
derivative sigmoid(PAD_LOGIT) is 0 as well; padded pass-through dims and padded value columns
are zeros.  Scores, outputs and the gradients of the real dims are therefore those of the
unpadded problem; the padding is built from differentiable torch ops, so autograd returns the
gradients of the real dims (and of freqs[..., :R], bias[..., :R]) by itself.  The softmax scale is
always passed explicitly by the callers (from the caller's D), never re-derived from the padded
width.
"""
from __future__ import annotations

from typing import NamedTuple, Optional

import torch
import torch.nn.functional as F
from torch import Tensor

PAD_LOGIT = -1.0e4   # fits fp16 / bf16 / fp32; softplus and sigmoid of it are exactly 0 in fp32


def _ceil8(n: int) -> int:
    return (n + 7) // 8 * 8


class PadPlan(NamedTuple):
    D: int    # caller's head dim
    R: int    # caller's rotate dim
    R8: int   # padded rotate dim
    Dp: int   # padded head dim


def pad_plan(D: int, R: int) -> Optional[PadPlan]:
    """None when D and R are multiples of 8 (the kernels take them as they are)."""
    if D % 8 == 0 and R % 8 == 0:
        return None
    R8 = _ceil8(R)
    return PadPlan(D, R, R8, R8 + _ceil8(D - R))


def pad_qk(t: Tensor, p: PadPlan) -> Tensor:
    """(.., D) query / key rows -> (.., Dp): rotated dims, PAD_LOGIT fill, pass-through dims, zeros."""
    lead = t.shape[:-1]
    parts = [t[..., :p.R]]
    if p.R8 > p.R:
        parts.append(t.new_full(lead + (p.R8 - p.R,), PAD_LOGIT))
    parts.append(t[..., p.R:])
    tail = p.Dp - p.R8 - (p.D - p.R)
    if tail:
        parts.append(t.new_zeros(lead + (tail,)))
    return torch.cat(parts, -1)


def unpad_qk(t: Tensor, p: PadPlan) -> Tensor:
    """(.., Dp) -> (.., D): the inverse selection of pad_qk (gradients of the real dims)."""
    return torch.cat([t[..., :p.R], t[..., p.R8:p.R8 + p.D - p.R]], -1)


def pad_last(t: Optional[Tensor], n: int) -> Optional[Tensor]:
    """Zeros appended to the last dim up to n (None passes through)."""
    if t is None or t.shape[-1] == n:
        return t
    return F.pad(t, (0, n - t.shape[-1]))
