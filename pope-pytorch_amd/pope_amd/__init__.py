"""pope_amd: PoPE attention for AMD Instinct MI355X (gfx950).

Drop-in for the public API of lucidrains/PoPE-pytorch (``PoPE_pytorch/__init__.py:1-11``):
``PoPE``, ``apply_pope_to_qk``, ``compute_attn_similarity``, ``flash_attn_with_pope``,
``AxialPoPE``.  GPU tensors run hand-written HIP kernels (libpope_hip.so, C ABI in
include/pope_abi.h) registered as ``torch.library`` ops under the ``pope_amd``
namespace.
"""
from .pope import PoPE, PolarEmbedReturn, apply_pope_to_qk
from .pope_nd import AxialPoPE
from .attention import compute_attn_similarity, compute_attn_similarity_non_fused, flash_attn_with_pope

__all__ = [
    "PoPE", "PolarEmbedReturn", "apply_pope_to_qk", "AxialPoPE",
    "compute_attn_similarity", "compute_attn_similarity_non_fused", "flash_attn_with_pope",
]
