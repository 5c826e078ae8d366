"""RMSNorm, AdaRMSNorm, SwiGLUMLPFused and RotaryEmbedding modules
(hydra/layers/common.py:74-338) with their arithmetic on the HIP kernels.
Parameter and buffer names match the reference (weight; gate_up.weight,
down.weight; _cond_proj; cos_cached, sin_cached)."""
from __future__ import annotations

from typing import Any, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _lib
from .._autograd import track
from ..kernels import fused_rms_norm, fused_rope, fused_swiglu


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight (common.py:74-118), fp32 inside,
    one rounding (the reference's module calls F.rms_norm, which rounds
    x * rsqrt(...) before the weight product; the two agree to the input
    dtype's precision)."""

    _hydra_norm_mode = _lib.NORM_RMS  # what hydra_residual_norm_fwd computes for it

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return fused_rms_norm(x, self.weight, self.eps)


def residual_norm(x: torch.Tensor, *, r: Optional[torch.Tensor] = None, alpha: float = 1.0,
                  b1: Optional[torch.Tensor] = None, b2: Optional[torch.Tensor] = None,
                  weight: Optional[torch.Tensor] = None, eps: float = 1e-6, norm: int = _lib.NORM_RMS,
                  want_h: bool = False) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """(h, y) with h = x + alpha * r + b1 + b2 (each add rounded to x's dtype
    as the reference's tensor ops are) and y = norm(h) (hydra_residual_norm_fwd:
    RMSNorm, AdaRMSNorm's input-dtype steps, or none).  x, r: [..., dim];
    b1, b2, weight: [dim].  Returns h only when want_h (or no norm)."""
    _lib.require_gpu("residual_norm", x, r, b1, b2, weight)
    dim = x.shape[-1]
    x2 = x.reshape(-1, dim)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    r2 = None
    if r is not None:
        if r.shape != x.shape:
            raise ValueError(f"residual_norm: r shape {tuple(r.shape)} != x shape {tuple(x.shape)}")
        r2 = r.to(x.dtype).reshape(-1, dim)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
    vecs = []
    for b in (b1, b2):
        if b is not None:
            b = b.reshape(-1).to(x.dtype).contiguous()
            if b.numel() != dim:
                raise ValueError("residual_norm: bias vectors must have dim elements")
        vecs.append(b)
    w = None
    if norm != _lib.NORM_NONE:
        if weight is None or weight.shape != (dim,):
            raise ValueError("residual_norm: the norm needs a [dim] weight")
        w = weight if weight.dtype in (x.dtype, torch.float32) else weight.to(x.dtype)
        w = w.contiguous()
    h = torch.empty((rows, dim), dtype=x.dtype, device=x.device) if (want_h or norm == _lib.NORM_NONE) else None
    y = torch.empty((rows, dim), dtype=x.dtype, device=x.device) if norm != _lib.NORM_NONE else None
    with torch.cuda.device(x.device):
        _lib.call("hydra_residual_norm_fwd", x2.data_ptr(), x2.stride(0), _lib.ptr(r2),
                  r2.stride(0) if r2 is not None else 0, float(alpha), _lib.ptr(vecs[0]),
                  _lib.ptr(vecs[1]), _lib.ptr(w), float(eps), int(norm), _lib.ptr(h), dim,
                  _lib.ptr(y), dim, rows, dim, _lib.dtype_code(x),
                  _lib.dtype_code(w) if w is not None else _lib.dtype_code(x), _lib.stream(x))
    shape = x.shape
    return (h.view(shape) if h is not None else None), (y.view(shape) if y is not None else None)


class AdaRMSNorm(nn.Module):
    """AdaRMSNorm (common.py:121-172).  The unconditioned forward is the
    reference's `_rmsnorm` computed in the input dtype, step for step
    (x.pow(2).mean, + eps, rsqrt, * x, * weight each rounded), on
    hydra_residual_norm_fwd; the conditioned path applies the learned
    scale/shift on top.  Forward only: a backward through it raises."""

    _hydra_norm_mode = _lib.NORM_ADA

    def __init__(self, dim: int, *, cond_dim: Optional[int] = None, eps: float = 1e-6, **_: Any):
        super().__init__()
        self.dim = dim
        self.cond_dim = cond_dim
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))
        self._cond_proj: Optional[nn.Linear]
        self._cond_proj = nn.Linear(cond_dim, 2 * dim) if cond_dim is not None else None

    def _rmsnorm(self, x: torch.Tensor) -> torch.Tensor:
        _, y = residual_norm(x, weight=self.weight, eps=self.eps, norm=_lib.NORM_ADA)
        return track(y, x, self.weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._rmsnorm(x)

    def forward_conditioned(self, x: torch.Tensor, cond: torch.Tensor) -> torch.Tensor:
        if self._cond_proj is None:
            raise RuntimeError("AdaRMSNorm was constructed without cond_dim; "
                               "conditioning is not available.")
        h = self._rmsnorm(x)
        s, b = self._cond_proj(cond).chunk(2, dim=-1)
        return h * (1.0 + s.unsqueeze(1)) + b.unsqueeze(1)


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

    def forward_residual(self, h: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """h + forward(x), with the residual add in the down projection's
        GEMM epilogue (one rounding instead of two)."""
        gate, up = F.linear(x, self.gate_up.weight).chunk(2, dim=-1)
        act = fused_swiglu(gate, up)
        dim = h.shape[-1]
        out = torch.addmm(h.reshape(-1, dim), act.reshape(-1, act.shape[-1]), self.down.weight.t())
        return out.view(h.shape)


SwiGLUMLP = SwiGLUMLPFused


class RotaryEmbedding(nn.Module):
    """RotaryEmbedding (common.py:242-338): the reference's fp32 cos/sin cache
    [1, 1, seq, head_dim/2] (theta `base`, optional `scaling_factor`), applied
    to interleaved pairs of [B, H, S, head_dim] by fused_rope."""

    def __init__(self, head_dim: int, max_seq_len: int = 8192, base: float = 10000.0,
                 scaling_factor: float = 1.0):
        super().__init__()
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.base = base
        self.scaling_factor = scaling_factor
        self._init_cache(max_seq_len)

    def _init_cache(self, seq_len: int) -> None:
        """common.py:268-285."""
        inv_freq = 1.0 / (self.base ** (torch.arange(0, self.head_dim, 2).float() / self.head_dim))
        if self.scaling_factor != 1.0:
            inv_freq = inv_freq / self.scaling_factor
        freqs = torch.outer(torch.arange(seq_len, dtype=torch.float32), inv_freq)
        self.register_buffer("cos_cached", freqs.cos()[None, None], persistent=False)
        self.register_buffer("sin_cached", freqs.sin()[None, None], persistent=False)
        self.max_seq_len = seq_len

    def extend_cache(self, seq_len: int) -> None:
        if seq_len > self.max_seq_len:
            device = self.cos_cached.device
            self._init_cache(seq_len)
            self.cos_cached = self.cos_cached.to(device)
            self.sin_cached = self.sin_cached.to(device)

    def forward(self, x: torch.Tensor, seq_len: Optional[int] = None) -> torch.Tensor:
        if seq_len is None:
            seq_len = x.shape[2]
        if self.cos_cached.device != x.device:
            self.cos_cached = self.cos_cached.to(x.device)
            self.sin_cached = self.sin_cached.to(x.device)
        if seq_len > self.max_seq_len:
            self.extend_cache(seq_len)
        return fused_rope(x, self.cos_cached[:, :, :seq_len, :], self.sin_cached[:, :, :seq_len, :])

    def get_cos_sin(self, seq_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if seq_len > self.max_seq_len:
            self.extend_cache(seq_len)
        return self.cos_cached[:, :, :seq_len, :], self.sin_cached[:, :, :seq_len, :]
