"""Oracle for hydra/kernels/fused_ops.py (CPU reference paths).

Test infrastructure only: see oracle/__init__.py.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """_rms_norm_pytorch (hydra/kernels/fused_ops.py:1196-1205): F.rms_norm."""
    return F.rms_norm(x, [x.shape[-1]], weight=weight, eps=eps)


def rms_norm_fp32(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """The Triton kernel's arithmetic (fused_ops.py:991-1007): fp32 sum of
    squares, x * rsqrt(mean + eps) * w in fp32, one rounding to x.dtype."""
    xf, wf = x.float(), weight.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * r * wf).to(x.dtype)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """_rope_pytorch (fused_ops.py:300-306), with the output cast back to
    x.dtype as the Triton path (fused_ops.py:270, empty_like) and the
    attention fallback (attention.py:195-199) both do.  cos/sin are
    [1,1,Smax,D/2] or [S,D/2]."""
    S = x.shape[2]
    if cos.dim() == 2:
        cos, sin = cos[None, None], sin[None, None]
    cos = cos[:, :, :S, :]
    sin = sin[:, :, :S, :]
    x1, x2 = x[..., ::2], x[..., 1::2]
    out = torch.stack([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1).flatten(-2)
    return out.to(x.dtype)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """_swiglu_pytorch (fused_ops.py:881-883): F.silu(gate) * up."""
    return F.silu(gate) * up


def swiglu_fp32(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """The Triton kernel's arithmetic (fused_ops.py:717-725): fp32 math, one
    rounding to the input dtype."""
    g = gate.float()
    return (g * torch.sigmoid(g) * up.float()).to(gate.dtype)


def qk_norm(q, k, scale: float, temperature: float = 1.0):
    """_qk_norm_pytorch (fused_ops.py:587-596): F.normalize (eps 1e-12)."""
    return (F.normalize(q, p=2, dim=-1) * scale,
            F.normalize(k, p=2, dim=-1) * scale * temperature)


def qk_norm_triton_formula(q, k, scale: float, temperature: float = 1.0):
    """The Triton kernel's arithmetic (fused_ops.py:347-369):
    x * rsqrt(sum(x^2) + 1e-8) * scale (* temperature for k), fp32, one
    rounding."""
    qf, kf = q.float(), k.float()
    qo = qf * torch.rsqrt(qf.pow(2).sum(-1, keepdim=True) + 1e-8) * scale
    ko = kf * torch.rsqrt(kf.pow(2).sum(-1, keepdim=True) + 1e-8) * scale * temperature
    return qo.to(q.dtype), ko.to(k.dtype)


def rope_cache(head_dim: int, max_seq_len: int, theta: float = 10000.0):
    """CCGQAAttention._init_rope (attention.py:160-185): fp32 cos/sin
    [1,1,max_seq_len,head_dim/2]."""
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    t = torch.arange(max_seq_len, dtype=torch.float32)
    ang = torch.outer(t, freqs)
    return ang.cos()[None, None], ang.sin()[None, None]
