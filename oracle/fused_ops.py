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


# ---------------------------------------------------------------------------
# Backward of the fused ops (the reference's PyTorch backward paths)
# ---------------------------------------------------------------------------
def rms_norm_backward(x: torch.Tensor, weight: torch.Tensor, grad_out: torch.Tensor,
                      eps: float = 1e-6):
    """_rms_norm_backward_pytorch (hydra/kernels/fused_ops.py:1251-1281), fp32
    inside: r = rsqrt(mean(x^2) + eps), x_norm = x * r;
    grad_w = clamp(sum over rows of x_norm * g, +-100) in weight.dtype;
    grad_x = clamp(g * w * r - x_norm * mean(g * w * x_norm), +-100) in x.dtype.
    The correction term is the reference's as written: the exact derivative
    has one more factor r in it (the two agree when mean(x^2) + eps = 1)."""
    dim = x.shape[-1]
    xf = x.reshape(-1, dim).float()
    wf = weight.float()
    gf = grad_out.reshape(-1, dim).float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    xn = xf * r
    grad_w = (xn * gf).sum(0).clamp(-100.0, 100.0).to(weight.dtype)
    corr = (gf * wf * xn).mean(-1, keepdim=True)
    grad_x = (gf * wf * r - xn * corr).clamp(-100.0, 100.0).to(x.dtype)
    return grad_x.view(x.shape), grad_w


def swiglu_backward(gate: torch.Tensor, up: torch.Tensor, grad_out: torch.Tensor):
    """_swiglu_backward_pytorch (fused_ops.py:926-948), fp32 inside:
    s = sigmoid(g); grad_gate = clamp(go * u * s * (1 + g * (1 - s)), +-100);
    grad_up = clamp(go * g * s, +-100); each in its input's dtype."""
    g, u, go = gate.float(), up.float(), grad_out.float()
    s = torch.sigmoid(g)
    grad_gate = (go * u * (s * (1.0 + g * (1.0 - s)))).clamp(-100.0, 100.0).to(gate.dtype)
    grad_up = (go * (g * s)).clamp(-100.0, 100.0).to(up.dtype)
    return grad_gate, grad_up


def qk_norm_backward(q: torch.Tensor, k: torch.Tensor, grad_q: torch.Tensor,
                     grad_k: torch.Tensor, scale: float, temperature: float = 1.0):
    """_qk_norm_backward_pytorch (fused_ops.py:638-672), fp32 inside, per
    row: n = max(||x||, 1e-6), xn = x / n,
    grad = clamp(s / n * (g - xn * <xn, g>), +-100) with s = scale for q and
    scale * temperature for k; in the inputs' dtype."""
    def one(x, gx, s):
        xf, gf = x.float(), gx.float()
        n = torch.norm(xf, p=2, dim=-1, keepdim=True).clamp(min=1e-6)
        xn = xf / n
        dot = (xn * gf).sum(-1, keepdim=True)
        return (s / n * (gf - xn * dot)).clamp(-100.0, 100.0).to(x.dtype)
    return one(q, grad_q, scale), one(k, grad_k, scale * temperature)


def rope_backward(grad_out: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Gradient of `rope` with respect to x, as autograd gives it through the
    reference's CPU path (_rope_pytorch, fused_ops.py:300-306; the Triton
    path records no gradient): each pair rotated back,
    (g1 c + g2 s, -g1 s + g2 c), fp32 inside, in grad_out.dtype."""
    S = grad_out.shape[2]
    if cos.dim() == 2:
        cos, sin = cos[None, None], sin[None, None]
    cos = cos[:, :, :S, :].float()
    sin = sin[:, :, :S, :].float()
    g = grad_out.float()
    g1, g2 = g[..., ::2], g[..., 1::2]
    out = torch.stack([g1 * cos + g2 * sin, -g1 * sin + g2 * cos], dim=-1).flatten(-2)
    return out.to(grad_out.dtype)


def chunked_cross_entropy(hidden, weight, targets, ignore_index=-100, grad_output=1.0):
    """fp64 restatement of ChunkedCrossEntropyFunction (fused_ops.py:1382-1531):
    logits = h W^T; when any target other than ignore_index lies outside
    [0, V), the whole target vector (ignore_index entries included) is
    clamped into [0, V) and validity is recomputed from it (:1407-1422,
    :1440-1441); loss = mean over valid tokens of logsumexp(x) - x[t]
    (0 with none); grad_x = (softmax(x) - onehot(t)) * grad_output / n_valid
    on valid rows, 0 on ignored rows; grad_h = grad_x W, grad_W = grad_x^T h.
    Returns (loss, grad_h, grad_W) in fp64.  Pinned against autograd of
    F.cross_entropy and against the reference's own outputs
    (tests/golden/chunked_ce_cpu.npz) in tests/test_oracle_pins.py."""
    dim = hidden.shape[-1]
    h = hidden.reshape(-1, dim).double()
    w = weight.double()
    t = targets.reshape(-1).long()
    V = w.shape[0]
    valid = t != ignore_index
    if bool((valid & ((t < 0) | (t >= V))).any()):
        t = t.clamp(0, V - 1)
        valid = t != ignore_index
    tc = torch.where(valid, t, torch.zeros_like(t))
    x = h @ w.t()
    lse = torch.logsumexp(x, -1)
    rows = lse - x.gather(1, tc[:, None])[:, 0]
    n = int(valid.sum())
    loss = (rows * valid).sum() / n if n else torch.zeros((), dtype=torch.float64)
    g = torch.softmax(x, -1)
    g[torch.arange(len(t)), tc] -= 1.0
    g = g * valid[:, None] * (grad_output / max(n, 1))
    return loss, (g @ w).view(hidden.shape), g.t() @ h


def token_losses_from_hidden(hidden, weight, targets, ignore_index=-100):
    """fp64 restatement of compute_token_losses_from_hidden
    (hydra/training/loop.py:28-89): per-token logsumexp(x) - x[t], 0 where
    the target is ignore_index; when some non-ignored target is out of
    [0, V), the whole target vector (ignore entries included) is clamped
    into [0, V) and validity recomputed (:54-70)."""
    B, L, D = hidden.shape
    w = weight.double()
    V = w.shape[0]
    h = hidden.reshape(-1, D).double()
    t = targets.reshape(-1).long().clone()
    valid = t != ignore_index
    vt = t[valid]
    if vt.numel() and ((vt < 0) | (vt >= V)).any():
        t = t.clamp(0, V - 1)
        valid = t != ignore_index
    x = h @ w.t()
    tc = torch.where(valid, t, torch.zeros_like(t))
    loss = torch.logsumexp(x, -1) - x.gather(1, tc[:, None])[:, 0]
    return (loss * valid).view(B, L)
