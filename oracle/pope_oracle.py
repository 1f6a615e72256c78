"""CPU oracle for the PoPE attention path -- TEST INFRASTRUCTURE ONLY.

This module restates, in plain CPU PyTorch, the reference's own PyTorch path for
PoPE (lucidrains/PoPE-pytorch v0.0.15).  It is the checker that the HIP kernels
are compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
(``pope_amd``) never does, and must fail loudly rather than fall back here.

Every function cites the reference file:line it follows.  All arithmetic runs
in the dtype of the tensors passed in (callers use float64 for pinning and
float32 to mirror the reference's fp32 rounding, e.g. ``fl(freqs + bias)``).

How each function is pinned (tests/test_oracle.py, tests/golden/):
  * ``inv_freqs`` / ``pope_freqs`` / ``axial_*``: closed forms
    (freqs[i, j] = i * theta**(-j/dim), reversed-axis grid order) and the
    shapes the reference's tests assert (test_readme.py:36,47).
  * ``clamp_bias``: closed form on values inside, at and beyond [-2 pi, 0] and
    the gradient torch's clamp passes (1 inside and at the bounds, 0 beyond).
  * ``softplus``: torch.nn.functional.softplus (beta 1, threshold 20) over
    [-100, 100] in float32 and float64, and golden inputs past the threshold.
  * ``_repeat_heads``: einops.repeat(t, 'b h ... -> b (g h) ...') -- the
    reference's own layout call (attention.py:44-45) -- and a golden case with
    Hq = 4, Hk = 2, where h % Hk and h // (Hq / Hk) differ.
  * ``apply_pope_to_qk``: interleave order and raw pass-through dims by
    construction checks, right-aligned query rows, output shapes of
    test_pope.py:21-29 / test_readme.py:18-24,54.
  * ``sim_nonfused``: float64 brute force of
    S_ij = sum_{d<R} a_id c_jd cos(phi_id - psi_jd) + sum_{d>=R} q_id k_jd
    (tests/golden/make_golden.py, an independent loop formula), translation
    invariance under ``offset``, R = 0 reducing to q k^T, and the phase identity
    sum_i dphi_i + sum_j dpsi_j = 0.
  * ``flash_nonfused``: float64 brute-force softmax attention with top-left
    causal AND key-padding masks (golden fixtures), fully-masked rows -> 0,
    and flash == softmax(scale * sim) V (reference test_flash_attn.py:78-110).
  * gradients: central finite differences in float64 on the golden cases.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = [
    "inv_freqs", "pope_freqs", "clamp_bias", "axial_inv_freqs", "axial_grid_positions",
    "axial_freqs", "softplus", "apply_pope_to_qk", "sim_nonfused", "flash_nonfused",
    "flash_lse",
]


def inv_freqs(dim: int, theta: float = 10000.0) -> torch.Tensor:
    """theta ** -(arange(dim) / dim) in fp32 -- pope.py:106-107 (dim frequencies, not dim/2)."""
    return theta ** -(torch.arange(dim).float() / dim)


def pope_freqs(pos_or_seq_len, inv: torch.Tensor, offset=0) -> torch.Tensor:
    """Outer product of positions and inverse frequencies -- pope.py:131-141."""
    if torch.is_tensor(pos_or_seq_len):
        pos = pos_or_seq_len
    else:
        pos = torch.arange(pos_or_seq_len, dtype=inv.dtype)
    pos = pos + offset
    return pos[..., :, None] * inv


def clamp_bias(bias: torch.Tensor) -> torch.Tensor:
    """Learned key phase bias clamped to [-2*pi, 0] -- pope.py:145, pope_nd.py:104."""
    return bias.clamp(-2.0 * math.pi, 0.0)


def axial_inv_freqs(axial_dims, theta: float = 10000.0):
    """Per-axis inverse frequencies -- pope_nd.py:48-52."""
    return [theta ** -(torch.arange(d).float() / d) for d in axial_dims]


def axial_grid_positions(*dims) -> torch.Tensor:
    """Grid positions, meshgrid 'ij' stacked in REVERSED axis order -- pope_nd.py:65-68.

    Column 0 of the result is the LAST axis (fastest varying)."""
    grid = torch.meshgrid(*[torch.arange(d).float() for d in dims], indexing="ij")
    return torch.stack([g.flatten() for g in reversed(grid)], dim=-1)


def axial_freqs(pos: torch.Tensor, invs) -> torch.Tensor:
    """Concatenation of per-axis outer products -- pope_nd.py:84-100."""
    assert pos.shape[-1] == len(invs)
    return torch.cat([pos[..., i, None] * inv for i, inv in enumerate(invs)], dim=-1)


def softplus(x: torch.Tensor) -> torch.Tensor:
    """F.softplus with beta=1, threshold=20 (x > 20 -> x) -- pope.py:34,60; triton_pope.py:18-20."""
    return torch.where(x > 20.0, x, torch.log1p(torch.exp(torch.clamp(x, max=20.0))))


def _slice_right(freqs: torch.Tensor, n: int) -> torch.Tensor:
    """Last ``n`` rows along dim -2: the right-aligned query phases (pope.py:64;
    the kernels' q_off = Nk - Nq, triton_pope_flash_attn.py:54)."""
    return freqs[..., freqs.shape[-2] - n:, :]


def apply_pope_to_qk(freqs, bias, q, k, return_complex: bool = False):
    """The materialising polar transform -- pope.py:30-86.

    q: (..., Nq, D), k: (..., Nk, D); freqs (N, R) / (B, N, R); bias (Hk or 1, R).
    Returns q_hat, k_hat of last dim D + R with the rotated part interleaved
    [a cos, a sin] per dim (pope.py:70,78) and the pass-through dims raw (pope.py:82-84).
    """
    q_len, k_len, qk_dim, rot = q.shape[-2], k.shape[-2], q.shape[-1], freqs.shape[-1]
    assert q_len <= k_len and rot <= qk_dim
    partial = rot < qk_dim
    if partial:
        q, q_rest = q[..., :rot], q[..., rot:]
        k, k_rest = k[..., :rot], k[..., rot:]
        if return_complex:
            q_rest = torch.polar(q_rest, torch.zeros_like(q_rest))
            k_rest = torch.polar(k_rest, torch.zeros_like(k_rest))
    if freqs.ndim == 3:
        freqs = freqs[:, None]                       # b n d -> b 1 n d  (pope.py:53-54)
    freqs_with_bias = freqs + bias[:, None, :]       # h d -> h 1 d      (pope.py:56)
    q, k = softplus(q), softplus(k)                  # pope.py:60
    fq = _slice_right(freqs, q_len)                  # pope.py:64
    if return_complex:
        q = torch.polar(q, fq.expand_as(q) if fq.shape != q.shape else fq)
        k = torch.polar(k, freqs_with_bias.expand_as(k) if freqs_with_bias.shape != k.shape else freqs_with_bias)
    else:
        q = torch.stack([q * fq.cos(), q * fq.sin()], dim=-1).flatten(-2)   # (d two)
        k = torch.stack([k * freqs_with_bias.cos(), k * freqs_with_bias.sin()], dim=-1).flatten(-2)
    if partial:
        q = torch.cat((q, q_rest), dim=-1)
        k = torch.cat((k, k_rest), dim=-1)
    return q, k


def _repeat_heads(t: torch.Tensor, groups: int) -> torch.Tensor:
    """einops 'b h ... -> b (g h) ...': query head i reads kv head i % Hk (attention.py:44-45)."""
    return t.repeat(1, groups, *([1] * (t.ndim - 2))) if groups > 1 else t


def sim_nonfused(q, k, freqs, bias):
    """Unscaled PoPE similarity -- attention.py:30-47. q (B,Hq,Nq,D), k (B,Hk,Nk,D)."""
    qh, kh = apply_pope_to_qk(freqs, bias, q, k)
    kh = _repeat_heads(kh, qh.shape[1] // kh.shape[1])
    return qh @ kh.transpose(-1, -2)


def _attn_mask(B, Nq, Nk, mask, causal, device):
    """Keep-mask (B,1,Nq,Nk): key padding (True = keep, attention.py:129-131) AND
    top-left causal (j <= i, SDPA's convention for is_causal, attention.py:133-138)."""
    keep = torch.ones(B, 1, Nq, Nk, dtype=torch.bool, device=device)
    if mask is not None:
        keep = keep & mask[:, None, None, :].bool()
    if causal:
        keep = keep & torch.ones(Nq, Nk, dtype=torch.bool, device=device).tril()
    return keep


def flash_nonfused(q, k, v, freqs=None, bias=None, mask=None, causal=False, softmax_scale=None):
    """PoPE attention -- attention.py:106-145 with the SDPA call written out.

    softmax(scale * q_hat k_hat^T + M) v, M = -inf where the explicit AND mask is
    False; a fully-masked row gives 0 (triton_pope_flash_attn.py:114).
    The output is returned in the dtype of the computation (callers cast)."""
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    if freqs is not None:
        qh, kh = apply_pope_to_qk(freqs, bias, q, k)
    else:
        qh, kh = q, k
    g = qh.shape[1] // kh.shape[1]
    kh, v = _repeat_heads(kh, g), _repeat_heads(v, g)
    v = v.to(qh.dtype)
    s = (qh @ kh.transpose(-1, -2)) * scale
    keep = _attn_mask(q.shape[0], q.shape[-2], k.shape[-2], mask, causal, q.device)
    s = s.masked_fill(~keep, float("-inf"))
    row_has = keep.any(-1, keepdim=True)
    p = torch.softmax(s.masked_fill(~row_has, 0.0), dim=-1) * row_has
    return p @ v


def flash_lse(q, k, freqs=None, bias=None, mask=None, causal=False, softmax_scale=None):
    """Natural-log log-sum-exp of the masked scaled scores per query row (B,Hq,Nq);
    -inf for fully-masked rows -- triton_pope_flash_attn.py:117."""
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    if freqs is not None:
        qh, kh = apply_pope_to_qk(freqs, bias, q, k)
    else:
        qh, kh = q, k
    kh = _repeat_heads(kh, qh.shape[1] // kh.shape[1])
    s = (qh @ kh.transpose(-1, -2)) * scale
    keep = _attn_mask(q.shape[0], q.shape[-2], k.shape[-2], mask, causal, q.device)
    return torch.logsumexp(s.masked_fill(~keep, float("-inf")), dim=-1)

