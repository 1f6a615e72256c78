"""PoPE attention entry points: fused HIP path for GPU tensors, torch path otherwise.

API mirror of the reference's ``PoPE_pytorch/attention.py``:
``compute_attn_similarity_non_fused`` (:30-47), ``compute_attn_similarity``
(:49-73) and ``flash_attn_with_pope`` (:75-145), with the same arguments,
defaults, layouts (``head_dimension_at_first``), asserts and return values.

Dispatch (reference :21-26, :63-71, :86): GPU tensors go to the HIP kernels of
libpope_hip.so; if that library is missing the call raises -- there is no silent
fallback.  Flash attention covers head dims up to 256 (after padding to a multiple of 8)
with its own kernels; wider heads run with the polar transform materialised on the
device (the polar transform kernel) and the attention products in fp32
(``_attend_materialised``).  The torch path (``fused=False`` or CPU tensors) is the reference's own
non-fused computation, with the key-padding and causal masks combined into one
explicit boolean mask so the result does not depend on the torch version's
handling of ``attn_mask`` together with ``is_causal`` (reference :133-138).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .pope import apply_pope_to_qk

# The fused path is the HIP library; "available" means a GPU is present.  Whether
# the library loads is checked on first use and failures raise.
HIP_AVAILABLE = torch.cuda.is_available()


def exists(v):
    return v is not None


def default(v, d):
    return v if exists(v) else d


def divisible_by(num, den):
    return (num % den) == 0


def _to_head_first(*ts):
    return tuple(t.transpose(1, 2) for t in ts)


# widest (padded) head dim of the fused flash kernels (the register-tiled kernels up to 128, the
# wide ones up to 256); flash_attn_with_pope takes wider heads through its materialising path
FLASH_MAX_HEAD_DIM = 256


def _flash_width(D, pos_emb):
    """Head dim the flash kernels would see: D, or its padded width when D or the rotate dim
    is not a multiple of 8 (pope_amd._pad)."""
    from ._pad import pad_plan
    R = pos_emb[0].shape[-1] if exists(pos_emb) and exists(pos_emb[0]) else 0
    plan = pad_plan(D, R)
    return D if plan is None else plan.Dp


def _repeat_heads(t, groups):
    """'b h ... -> b (g h) ...': query head i reads kv head i % Hk."""
    return t.repeat(1, groups, *([1] * (t.ndim - 2))) if groups > 1 else t


def _keep_mask(mask, causal, Nq, Nk, device):
    keep = None
    if exists(mask):
        keep = mask.bool()[:, None, None, :]
    if causal:
        tri = torch.ones(Nq, Nk, dtype=torch.bool, device=device).tril()
        keep = tri if keep is None else keep & tri
    return keep


def _attend_materialised(q, k, v, pos_emb, mask, causal, softmax_scale):
    """Head-first PoPE attention for heads wider than the flash kernels cover (above 256): q_hat, k_hat from
    apply_pope_to_qk (the polar transform kernel for GPU tensors), then the masked softmax
    attention of attention.py:106-145 with the scores and the value product in fp32 (explicit
    products with contiguous right operands).  A row with every key masked gives 0."""
    out_dtype = v.dtype
    if exists(pos_emb):
        q, k = apply_pope_to_qk(pos_emb, q, k, to_magnitude=F.softplus)
    groups = q.shape[1] // k.shape[1]
    # repeated after the fp32 conversion, so the group heads' dk / dv are summed in fp32 and
    # rounded to the input dtype once
    qf, kf, vf = q.float(), k.float(), v.float()
    kf, vf = _repeat_heads(kf, groups), _repeat_heads(vf, groups)
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * softmax_scale
    keep = _keep_mask(mask, causal, q.shape[-2], k.shape[-2], q.device)
    if exists(keep):
        s = s.masked_fill(~keep, float("-inf"))
        row_any = keep.any(-1, keepdim=True)
        p = torch.softmax(s.masked_fill(~row_any, 0.0), dim=-1) * row_any
    else:
        p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vf).to(out_dtype)


def compute_attn_similarity_non_fused(q, k, pope, head_dimension_at_first=True):
    if not head_dimension_at_first:
        q, k = _to_head_first(q, k)
    q, k = apply_pope_to_qk(pope, q, k, to_magnitude=F.softplus)
    k = _repeat_heads(k, q.shape[1] // k.shape[1])
    return q @ k.transpose(-1, -2)


def compute_attn_similarity(q, k, pope, allow_tf32=True, head_dimension_at_first=True):
    assert divisible_by(q.shape[1 if head_dimension_at_first else 2], k.shape[1 if head_dimension_at_first else 2])
    freqs, bias = pope
    head_dim = q.shape[-1]
    assert head_dim in {32, 48, 64, 128, 256}, f"head_dim {head_dim} not in common sizes"

    is_cuda = q.is_cuda and k.is_cuda and freqs.is_cuda and bias.is_cuda
    if is_cuda:
        from .hip_pope import hip_compute_qk_similarity
        if not head_dimension_at_first:
            q, k = _to_head_first(q, k)
        return hip_compute_qk_similarity(q, k, freqs, bias, freqs.shape[-1], allow_tf32=allow_tf32)

    return compute_attn_similarity_non_fused(q, k, pope, head_dimension_at_first=head_dimension_at_first)


def flash_attn_with_pope(q, k, v, pos_emb=None, mask=None, causal=False, softmax_scale=None, fused=None,
                         head_dimension_at_first=True):
    fused = default(fused, q.is_cuda)
    softmax_scale = default(softmax_scale, q.shape[-1] ** -0.5)
    wide = fused and _flash_width(q.shape[-1], pos_emb) > FLASH_MAX_HEAD_DIM

    if wide:
        # heads wider than the flash kernels cover: the polar transform materialised on the device
        if not head_dimension_at_first:
            q, k, v = _to_head_first(q, k, v)
        out = _attend_materialised(q, k, v, pos_emb, mask, causal, softmax_scale)
        return out.transpose(1, 2) if not head_dimension_at_first else out

    if fused:
        from .hip_pope_flash_attn import flash_attn_head_first
        if not head_dimension_at_first:
            q, k, v = _to_head_first(q, k, v)
        freqs, bias = pos_emb if exists(pos_emb) else (None, None)
        out = flash_attn_head_first(q, k, v, freqs, bias, mask=mask, causal=causal, softmax_scale=softmax_scale)
        if not head_dimension_at_first:
            out = out.transpose(1, 2)
        return out

    # non-fused torch path, standardised to (batch, heads, seq, dim)
    if not head_dimension_at_first:
        q, k, v = _to_head_first(q, k, v)
    if exists(pos_emb):
        q, k = apply_pope_to_qk(pos_emb, q, k, to_magnitude=F.softplus)
    groups = q.shape[1] // k.shape[1]
    k, v = _repeat_heads(k, groups), _repeat_heads(v, groups)

    v_dtype = v.dtype
    if q.dtype != v.dtype:
        v = v.to(q.dtype)

    keep = _keep_mask(mask, causal, q.shape[-2], k.shape[-2], q.device)
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=keep, scale=softmax_scale)
    if exists(keep):
        # rows with every key masked give 0, as the fused kernels do
        row_any = keep.any(-1, keepdim=True)
        out = torch.where(row_any, out, torch.zeros((), dtype=out.dtype, device=out.device))
    out = out.to(v_dtype)

    if not head_dimension_at_first:
        out = out.transpose(1, 2)
    return out
