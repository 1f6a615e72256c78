"""PoPE frequencies, learned phase bias and the materialising polar transform.

API mirror of the reference's ``PoPE_pytorch/pope.py`` (PolarEmbedReturn :18,
apply_pope_to_qk :30-86, PoPE :90-147): same names, keyword arguments,
state_dict keys (``inv_freqs`` buffer, ``bias`` parameter) and error behaviour
(``AssertionError`` for q longer than k or a rotate dim above the head dim).

Two reference defects are fixed and documented:
  * ``bias_uniform_init=True`` raised because it called an in-place op on a
    leaf Parameter (pope.py:115-116); it now initialises under ``no_grad``.
  * ``inv_freqs`` typed ``list[float]`` was passed to ``register_buffer``
    unconverted (pope.py:100,109); lists are converted to a float tensor.
"""
from __future__ import annotations

from collections import namedtuple
from math import pi

import torch
import torch.nn.functional as F
from torch import Tensor, is_tensor
from torch.amp import autocast
from torch.nn import Module, Parameter

PolarEmbedReturn = namedtuple("PolarEmbedReturn", ("freqs", "bias"))


def exists(v):
    return v is not None


def _last_rows(t: Tensor, n: int) -> Tensor:
    """The last ``n`` entries along dim -2 (right-aligned query phases, pope.py:64)."""
    return t.narrow(-2, t.shape[-2] - n, n)


def _interleave(c: Tensor, s: Tensor) -> Tensor:
    """[c0, s0, c1, s1, ...] along the last dim ('two ... d -> ... (d two)', pope.py:70)."""
    return torch.stack((c, s), dim=-1).flatten(-2)


@autocast("cuda", enabled=False)
def apply_pope_to_qk(pope: PolarEmbedReturn, q: Tensor, k: Tensor, to_magnitude=F.softplus,
                     return_complex: bool = False):
    """Materialising polar transform (pope.py:30-86).

    q: (..., Nq, D), k: (..., Nk, D); pope.freqs (Nk, R) or (B, Nk, R); pope.bias
    (Hk, R) already clamped.  Returns (q_hat, k_hat) with last dim D + R: the
    first 2R columns interleave (m cos th, m sin th) per rotated dim, the
    remaining D - R pass-through dims are raw.  With ``return_complex`` the
    rotated dims come back as complex polar numbers (pass-through dims as
    complex with zero phase).
    """
    freqs, bias = pope
    q_len, k_len, qk_dim, rot = q.shape[-2], k.shape[-2], q.shape[-1], freqs.shape[-1]
    assert q_len <= k_len and rot <= qk_dim

    if q.is_cuda:
        from . import hip_polar
        if hip_polar.fits(q, k, freqs, bias, to_magnitude, return_complex):
            return hip_polar.polar(q, k, freqs, bias, return_complex)

    partial = rot < qk_dim
    if partial:
        q, q_rest = q[..., :rot], q[..., rot:]
        k, k_rest = k[..., :rot], k[..., rot:]
        if return_complex:
            q_rest = torch.polar(q_rest, torch.zeros_like(q_rest))
            k_rest = torch.polar(k_rest, torch.zeros_like(k_rest))

    if freqs.ndim == 3:
        freqs = freqs.unsqueeze(1)                    # b n d -> b 1 n d
    key_phase = freqs + bias.unsqueeze(-2)            # h d -> h 1 d

    q, k = to_magnitude(q), to_magnitude(k)
    q_phase = _last_rows(freqs, q_len)

    if return_complex:
        q = torch.polar(q, q_phase.expand(q.shape) if q_phase.shape != q.shape else q_phase)
        k = torch.polar(k, key_phase.expand(k.shape) if key_phase.shape != k.shape else key_phase)
    else:
        q = _interleave(q * q_phase.cos(), q * q_phase.sin())
        k = _interleave(k * key_phase.cos(), k * key_phase.sin())

    if partial:
        q = torch.cat((q, q_rest), dim=-1)
        k = torch.cat((k, k_rest), dim=-1)
    return q, k


class _ClampBias(torch.autograd.Function):
    """bias.clamp(lo, hi) with the gradient of torch's clamp (passed where lo <= bias <= hi, bounds included;
    zero outside and for NaN), in three launches per forward + backward instead of five: the forward saves
    the keep mask (clamped == bias) and the backward is one multiply."""

    @staticmethod
    def forward(ctx, bias, lo, hi):
        out = bias.clamp(lo, hi)
        ctx.save_for_backward(out == bias)
        return out

    @staticmethod
    def backward(ctx, grad):
        (keep,) = ctx.saved_tensors
        return grad * keep, None, None


class PoPE(Module):
    """Frequencies ``theta ** -(j / dim)`` for j < dim (pope.py:106-107) and a learned
    per-head key phase bias clamped to [-2 pi, 0] (pope.py:113,145)."""

    apply_pope_to_qk = staticmethod(apply_pope_to_qk)

    def __init__(self, dim, *, heads, theta=10000, bias_uniform_init=False,
                 inv_freqs: Tensor | list[float] | None = None):
        super().__init__()
        if not exists(inv_freqs):
            inv_freqs = theta ** -(torch.arange(dim).float() / dim)
        elif not is_tensor(inv_freqs):
            inv_freqs = torch.tensor(inv_freqs, dtype=torch.float32)
        self.register_buffer("inv_freqs", inv_freqs)
        self.bias = Parameter(torch.zeros(heads, dim))
        if bias_uniform_init:
            with torch.no_grad():
                self.bias.uniform_(-2.0 * pi, 0.0)

    @property
    def device(self):
        return self.inv_freqs.device

    @autocast("cuda", enabled=False)
    def forward(self, pos_or_seq_len: Tensor | int, offset=0) -> PolarEmbedReturn:
        if is_tensor(pos_or_seq_len):
            pos = pos_or_seq_len
        else:
            pos = torch.arange(pos_or_seq_len, device=self.device, dtype=self.inv_freqs.dtype)
        if is_tensor(offset) or offset != 0:   # adding an integer 0 would only copy pos (one launch)
            pos = pos + offset
        freqs = pos.unsqueeze(-1) * self.inv_freqs          # '... i, j -> ... i j'
        bias = _ClampBias.apply(self.bias, -2.0 * pi, 0.0) if self.bias.requires_grad else self.bias.clamp(-2.0 * pi, 0.0)
        return PolarEmbedReturn(freqs, bias)
