"""Axial (N-D) PoPE: per-axis frequencies concatenated over a position grid.

API mirror of the reference's ``PoPE_pytorch/pope_nd.py`` (AxialPoPE :23-106):
same constructor, ``get_grid_positions`` with the axes stacked in REVERSED order
(column 0 = last axis, pope_nd.py:68), ``inv_freqs.{i}`` parameters with
``requires_grad=False`` (:48-52) and the clamped ``bias`` (:56,104), so reference
checkpoints load unchanged.  ``bias_uniform_init=True`` initialises under
``no_grad`` (the reference raises, :58-59).
"""
from __future__ import annotations

from math import pi

import torch
from torch import Tensor
from torch.amp import autocast
from torch.nn import Module, Parameter, ParameterList

from .pope import PolarEmbedReturn, _ClampBias, apply_pope_to_qk


class AxialPoPE(Module):
    apply_pope_to_qk = staticmethod(apply_pope_to_qk)

    def __init__(self, dim, *, heads, axial_dims: tuple[int, ...] | None = None, theta=10000,
                 bias_uniform_init=False):
        super().__init__()
        self.dim = dim
        self.heads = heads
        if axial_dims is None:
            axial_dims = (dim,)
        self.axial_dims = axial_dims
        assert sum(axial_dims) == dim, f"sum of axial_dims {axial_dims} must be equal to dim {dim}"
        self.inv_freqs = ParameterList()
        for axial_dim in axial_dims:
            inv = theta ** -(torch.arange(axial_dim).float() / axial_dim)
            self.inv_freqs.append(Parameter(inv, requires_grad=False))
        self.bias = Parameter(torch.zeros(heads, dim))
        if bias_uniform_init:
            with torch.no_grad():
                self.bias.uniform_(-2.0 * pi, 0.0)

    @property
    def device(self):
        return self.bias.device

    @staticmethod
    def get_grid_positions(*dims, device=None) -> Tensor:
        grid = torch.meshgrid(*[torch.arange(d, device=device).float() for d in dims], indexing="ij")
        return torch.stack([g.flatten() for g in reversed(grid)], dim=-1)

    @autocast("cuda", enabled=False)
    def forward(self, pos_or_dims: Tensor | tuple[int, ...]) -> PolarEmbedReturn:
        if isinstance(pos_or_dims, tuple):
            pos = self.get_grid_positions(*pos_or_dims, device=self.device)
        else:
            pos = pos_or_dims
        assert pos.shape[-1] == len(self.axial_dims)
        freqs = torch.cat([pos[..., i, None] * inv for i, inv in enumerate(self.inv_freqs)], dim=-1)
        bias = _ClampBias.apply(self.bias, -2.0 * pi, 0.0) if self.bias.requires_grad else self.bias.clamp(-2.0 * pi, 0.0)
        return PolarEmbedReturn(freqs, bias)
