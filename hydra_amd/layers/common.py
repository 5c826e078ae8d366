"""RMSNorm and SwiGLUMLPFused modules (hydra/layers/common.py:74-118, 208-230)
with their elementwise parts on the HIP kernels.  Parameter names match the
reference (weight; gate_up.weight, down.weight)."""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels import fused_rms_norm, fused_swiglu


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight (common.py:74-118)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return fused_rms_norm(x, self.weight, self.eps)


class SwiGLUMLPFused(nn.Module):
    """down(silu(gate) * up) with [gate; up] = gate_up(x), first half = gate
    (common.py:208-230)."""

    def __init__(self, dim: int, hidden_dim: int):
        super().__init__()
        self.gate_up = nn.Linear(dim, 2 * hidden_dim, bias=False)
        self.down = nn.Linear(hidden_dim, dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = F.linear(x, self.gate_up.weight).chunk(2, dim=-1)
        return F.linear(fused_swiglu(gate, up), self.down.weight)
