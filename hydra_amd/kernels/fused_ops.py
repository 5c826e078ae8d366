"""Fused RMSNorm / RoPE / SwiGLU / QK-norm on MI355X.

Drop-in for hydra/kernels/fused_ops.py: same function names, signatures,
flags and error behaviour; the Triton kernels are replaced by the gfx950 HIP
kernels of libhydra_amd.so.  The flag names keep the reference's
"TRITON" spelling so callers need no change; here they mean "the HIP
library is loaded".

Autograd: RMSNorm, SwiGLU and QK-norm are autograd Functions whose backward
runs the HIP backward kernels (the reference's fused backward, same
formulas, clamps and flags); RoPE, which the reference's Triton path leaves
untracked, gets the gradient autograd gives through its CPU path, also on
the GPU.
"""
from __future__ import annotations

import os
from typing import Tuple

import torch
import torch.nn.functional as F

from .. import _lib

try:
    from torch.compiler import disable as compiler_disable
except ImportError:  # pragma: no cover
    def compiler_disable(fn):
        return fn

# ---------------------------------------------------------------------------
# Feature flags (fused_ops.py:60-94)
# ---------------------------------------------------------------------------
TRITON_AVAILABLE = _lib.available()
HIP_AVAILABLE = TRITON_AVAILABLE
TRITON_VERSION = (0, 0)


def _env_on(name: str, default: str) -> bool:
    return os.environ.get(name, default) == "1"


USE_TRITON_KERNELS = TRITON_AVAILABLE and os.environ.get("HYDRA_DISABLE_TRITON", "0") != "1"
USE_FUSED_ROPE = USE_TRITON_KERNELS and _env_on("HYDRA_ENABLE_FUSED_ROPE", "1") and not _env_on("HYDRA_DISABLE_FUSED_ROPE", "0")
USE_FUSED_QK_NORM = USE_TRITON_KERNELS
USE_FUSED_SWIGLU = USE_TRITON_KERNELS
USE_FUSED_RMS_NORM = USE_TRITON_KERNELS and _env_on("HYDRA_ENABLE_FUSED_RMS_NORM", "1") and not _env_on("HYDRA_DISABLE_FUSED_RMS_NORM", "0")
# Fused backward switches (fused_ops.py:80-94): default on, env overrides.
def _bwd_flags(enabled: bool):
    return (enabled and _env_on("HYDRA_ENABLE_FUSED_SWIGLU_BWD", "1") and not _env_on("HYDRA_DISABLE_FUSED_SWIGLU_BWD", "0"),
            enabled and _env_on("HYDRA_ENABLE_FUSED_RMS_NORM_BWD", "1") and not _env_on("HYDRA_DISABLE_FUSED_RMS_NORM_BWD", "0"),
            enabled and _env_on("HYDRA_ENABLE_FUSED_QK_NORM_BWD", "1") and not _env_on("HYDRA_DISABLE_FUSED_QK_NORM_BWD", "0"))


USE_FUSED_SWIGLU_BACKWARD, USE_FUSED_RMS_NORM_BACKWARD, USE_FUSED_QK_NORM_BACKWARD = _bwd_flags(USE_TRITON_KERNELS)
LIGER_CE_AVAILABLE = False
USE_LIGER_CE = False


def set_use_triton_kernels(enabled: bool) -> None:
    """Enable or disable the fused kernels globally (fused_ops.py:121-146).

    Raises RuntimeError when enabling without the HIP library, as the
    reference does without Triton.  While disabled, the fused_* functions
    raise instead of running: this build has no non-HIP path."""
    global USE_TRITON_KERNELS, USE_FUSED_ROPE, USE_FUSED_QK_NORM, USE_FUSED_SWIGLU, USE_FUSED_RMS_NORM
    global USE_FUSED_SWIGLU_BACKWARD, USE_FUSED_RMS_NORM_BACKWARD, USE_FUSED_QK_NORM_BACKWARD
    if enabled and not TRITON_AVAILABLE:
        raise RuntimeError("hydra_amd HIP library is not available (build it with __graft_entry__.build())")
    USE_TRITON_KERNELS = bool(enabled)
    USE_FUSED_ROPE = USE_TRITON_KERNELS and _env_on("HYDRA_ENABLE_FUSED_ROPE", "1") and not _env_on("HYDRA_DISABLE_FUSED_ROPE", "0")
    USE_FUSED_QK_NORM = USE_TRITON_KERNELS
    USE_FUSED_SWIGLU = USE_TRITON_KERNELS
    USE_FUSED_RMS_NORM = USE_TRITON_KERNELS and _env_on("HYDRA_ENABLE_FUSED_RMS_NORM", "1") and not _env_on("HYDRA_DISABLE_FUSED_RMS_NORM", "0")
    USE_FUSED_SWIGLU_BACKWARD, USE_FUSED_RMS_NORM_BACKWARD, USE_FUSED_QK_NORM_BACKWARD = _bwd_flags(USE_TRITON_KERNELS)


def get_kernel_status() -> dict:
    """Same keys as fused_ops.py:151-166 (plus the backend name)."""
    return {
        "backend": "hip-gfx950",
        "triton_available": TRITON_AVAILABLE,
        "triton_version": "N/A",
        "use_triton_kernels": USE_TRITON_KERNELS,
        "fused_rope": USE_FUSED_ROPE,
        "fused_qk_norm": USE_FUSED_QK_NORM,
        "fused_qk_norm_backward": USE_FUSED_QK_NORM_BACKWARD,
        "fused_swiglu": USE_FUSED_SWIGLU,
        "fused_swiglu_backward": USE_FUSED_SWIGLU_BACKWARD,
        "fused_rms_norm": USE_FUSED_RMS_NORM,
        "fused_rms_norm_backward": USE_FUSED_RMS_NORM_BACKWARD,
        "liger_ce_available": LIGER_CE_AVAILABLE,
        "use_liger_ce": USE_LIGER_CE,
    }


def _enabled(flag: bool, name: str) -> None:
    if not flag:
        raise RuntimeError(
            f"{name}: the fused HIP kernel is disabled (set_use_triton_kernels / "
            "HYDRA_DISABLE_* env) and this build has no other path")




# ---------------------------------------------------------------------------
# 1. RoPE (fused_ops.py:240-297)
# ---------------------------------------------------------------------------
def _rope_cache_2d(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    S, D = x.shape[2], x.shape[3]
    if cos.dim() == 4:
        cos = cos[0, 0, :S, :]
        sin = sin[0, 0, :S, :]
    if cos.shape[0] < S or cos.shape[-1] != D // 2:
        raise ValueError(f"fused_rope: cos/sin shape {tuple(cos.shape)} does not cover S={S}, D/2={D // 2}")
    if cos.stride(-1) != 1:
        cos = cos.contiguous()
    if sin.stride(-1) != 1 or sin.stride(0) != cos.stride(0):
        sin = sin.contiguous()
        cos = cos.contiguous()
    if sin.dtype != cos.dtype:
        sin = sin.to(cos.dtype)
    return cos, sin


def _rope_call(entry: str, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    B, H, S, D = x.shape
    if x.stride(-1) != 1:
        x = x.contiguous()
    out = torch.empty((B, H, S, D), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call(entry, x.data_ptr(), cos.data_ptr(), sin.data_ptr(), out.data_ptr(),
                  B, H, S, D, _lib.strides(x), cos.stride(0), _lib.dtype_code(x),
                  _lib.dtype_code(cos), _lib.stream(x))
    return out


class _RoPEFunction(torch.autograd.Function):
    """Forward hydra_rope_fwd; backward hydra_rope_bwd (the rotation's
    transpose), i.e. the gradient autograd gives through the reference's
    CPU path (_rope_pytorch, fused_ops.py:300-306)."""

    @staticmethod
    def forward(ctx, x, cos, sin):
        ctx.save_for_backward(cos, sin)
        return _rope_call("hydra_rope_fwd", x, cos, sin)

    @staticmethod
    def backward(ctx, grad_out):
        cos, sin = ctx.saved_tensors
        return _rope_call("hydra_rope_bwd", grad_out, cos, sin), None, None


@compiler_disable
def fused_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotary embedding on interleaved pairs.

    x: [B, n_heads, S, head_dim] (any strides); cos/sin: [1, 1, Smax, hd/2]
    or [S, hd/2].  Returns a contiguous tensor of x's shape and dtype."""
    _enabled(USE_FUSED_ROPE, "fused_rope")
    _lib.require_gpu("fused_rope", x, cos, sin)
    cos, sin = _rope_cache_2d(x, cos, sin)
    return _RoPEFunction.apply(x, cos, sin)


# ---------------------------------------------------------------------------
# 2. QK-norm (fused_ops.py:474-545)
# ---------------------------------------------------------------------------
class _QKNormFunction(torch.autograd.Function):
    """FusedQKNormFunction (fused_ops.py:496-545): forward hydra_qk_norm_fwd,
    backward hydra_qk_norm_bwd."""

    @staticmethod
    def forward(ctx, q, k, scale, temperature):
        qc, kc = q.contiguous(), k.contiguous()
        qo, ko = torch.empty_like(qc), torch.empty_like(kc)
        hd = q.shape[-1]
        with torch.cuda.device(q.device):
            _lib.call("hydra_qk_norm_fwd", qc.data_ptr(), kc.data_ptr(), qo.data_ptr(), ko.data_ptr(),
                      qc.numel() // hd, kc.numel() // hd, hd, float(scale), float(temperature),
                      _lib.dtype_code(q), _lib.stream(q))
        ctx.save_for_backward(qc, kc)
        ctx.scale, ctx.temperature = float(scale), float(temperature)
        return qo, ko

    @staticmethod
    def backward(ctx, grad_q_out, grad_k_out):
        _enabled(USE_FUSED_QK_NORM_BACKWARD, "fused_qk_norm backward")
        q, k = ctx.saved_tensors
        gqo = torch.zeros_like(q) if grad_q_out is None else grad_q_out.to(q.dtype).contiguous()
        gko = torch.zeros_like(k) if grad_k_out is None else grad_k_out.to(k.dtype).contiguous()
        gq, gk = torch.empty_like(q), torch.empty_like(k)
        hd = q.shape[-1]
        with torch.cuda.device(q.device):
            _lib.call("hydra_qk_norm_bwd", q.data_ptr(), k.data_ptr(), gqo.data_ptr(), gko.data_ptr(),
                      gq.data_ptr(), gk.data_ptr(), q.numel() // hd, k.numel() // hd, hd, ctx.scale,
                      ctx.temperature, _lib.dtype_code(q), _lib.stream(q))
        return gq, gk, None, None


@compiler_disable
def fused_qk_norm(q: torch.Tensor, k: torch.Tensor, scale: float,
                  temperature: float = 1.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """q * rsqrt(sum q^2 + 1e-8) * scale and k * rsqrt(sum k^2 + 1e-8) *
    scale * temperature over the last dim."""
    _enabled(USE_FUSED_QK_NORM, "fused_qk_norm")
    _lib.require_gpu("fused_qk_norm", q, k)
    if q.dtype != k.dtype or q.shape[-1] != k.shape[-1]:
        raise ValueError("fused_qk_norm: q and k must share dtype and head_dim")
    return _QKNormFunction.apply(q, k, scale, temperature)


# ---------------------------------------------------------------------------
# 3. SwiGLU (fused_ops.py:808-862)
# ---------------------------------------------------------------------------
def _rows_view(t: torch.Tensor):
    """(rows, row_stride) when t is a 2-D-collapsible view with unit stride on
    the last dim (e.g. one half of a gate_up.chunk(2)); else None."""
    if t.dim() == 0 or t.stride(-1) != 1:
        return None
    if t.dim() == 1:
        return 1, t.shape[-1]
    rs = t.stride(-2)
    rows = 1
    expect = rs
    for d in range(t.dim() - 2, -1, -1):
        if t.shape[d] != 1 and t.stride(d) != expect:
            return None
        rows *= t.shape[d]
        expect = expect * t.shape[d]
    return rows, rs


def _as_rows(t: torch.Tensor):
    """t (or a contiguous copy when its layout does not collapse to rows)
    with its (rows, row_stride)."""
    v = _rows_view(t)
    if v is None:
        t = t.contiguous()
        v = _rows_view(t)
    return t, v


class _SwiGLUFunction(torch.autograd.Function):
    """FusedSwiGLUFunction (fused_ops.py:823-862): forward hydra_swiglu_fwd,
    backward hydra_swiglu_bwd; gate/up may be the halves of one gate_up."""

    @staticmethod
    def forward(ctx, gate, up):
        gate, gv = _as_rows(gate)
        up, uv = _as_rows(up)
        hidden = gate.shape[-1] if gate.dim() else 1
        out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
        with torch.cuda.device(gate.device):
            _lib.call("hydra_swiglu_fwd", gate.data_ptr(), up.data_ptr(), out.data_ptr(),
                      gv[0], hidden, gv[1], uv[1], hidden, _lib.dtype_code(gate), _lib.stream(gate))
        ctx.save_for_backward(gate, up)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        _enabled(USE_FUSED_SWIGLU_BACKWARD, "fused_swiglu backward")
        gate, up = ctx.saved_tensors
        _, gv = _as_rows(gate)
        _, uv = _as_rows(up)
        go, ov = _as_rows(grad_out.to(gate.dtype))
        hidden = gate.shape[-1] if gate.dim() else 1
        gg = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
        gu = torch.empty(up.shape, dtype=up.dtype, device=up.device)
        with torch.cuda.device(gate.device):
            _lib.call("hydra_swiglu_bwd", gate.data_ptr(), up.data_ptr(), go.data_ptr(), gg.data_ptr(),
                      gu.data_ptr(), gv[0], hidden, gv[1], uv[1], ov[1], hidden, hidden,
                      _lib.dtype_code(gate), _lib.stream(gate))
        return gg, gu


@compiler_disable
def fused_swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up.  gate/up may be the strided halves of one gate_up
    tensor; they are read in place (no contiguous copies)."""
    _enabled(USE_FUSED_SWIGLU, "fused_swiglu")
    _lib.require_gpu("fused_swiglu", gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("fused_swiglu: gate and up must have the same shape and dtype")
    return _SwiGLUFunction.apply(gate, up)


# ---------------------------------------------------------------------------
# 4. RMSNorm (fused_ops.py:1114-1172)
# ---------------------------------------------------------------------------
def _norm_weight(weight: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """The weight as the kernels take it: x's dtype, or fp32 (an fp32 master
    weight is read in fp32, as the reference's kernel loads it,
    fused_ops.py:994); other dtypes are converted to x's."""
    w = weight if weight.dtype in (x.dtype, torch.float32) else weight.to(x.dtype)
    return w.contiguous()


class _RMSNormFunction(torch.autograd.Function):
    """FusedRMSNormFunction (fused_ops.py:1135-1172): forward
    hydra_rms_norm_fwd (hydra_residual_norm_fwd for an fp32 weight with a
    16-bit x), backward hydra_rms_norm_bwd.  An fp32 weight is used in fp32
    and its gradient written in fp32 (the reference's fp32 sum,
    :1244-1246)."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        dim = x.shape[-1]
        w = _norm_weight(weight, x)
        x, xv = _as_rows(x)
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        with torch.cuda.device(x.device):
            if w.dtype == x.dtype:
                _lib.call("hydra_rms_norm_fwd", x.data_ptr(), w.data_ptr(), out.data_ptr(),
                          xv[0], dim, xv[1], dim, float(eps), _lib.dtype_code(x), _lib.stream(x))
            else:
                _lib.call("hydra_residual_norm_fwd", x.data_ptr(), xv[1], None, 0, 1.0, None, None,
                          w.data_ptr(), float(eps), _lib.NORM_RMS, None, 0, out.data_ptr(), dim,
                          xv[0], dim, _lib.dtype_code(x), _lib.dtype_code(w), _lib.stream(x))
        ctx.save_for_backward(x, w)
        ctx.eps = float(eps)
        ctx.w_dtype = weight.dtype
        return out

    @staticmethod
    def backward(ctx, grad_out):
        _enabled(USE_FUSED_RMS_NORM_BACKWARD, "fused_rms_norm backward")
        x, w = ctx.saved_tensors
        dim = x.shape[-1]
        _, xv = _as_rows(x)
        go, ov = _as_rows(grad_out.to(x.dtype))
        gx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        gw = torch.empty((dim,), dtype=w.dtype, device=x.device)
        with torch.cuda.device(x.device):
            need = _lib.query("hydra_rms_norm_bwd_workspace", xv[0], dim)
            ws = _lib.scratch(need, x)
            _lib.call("hydra_rms_norm_bwd", x.data_ptr(), w.data_ptr(), go.data_ptr(), gx.data_ptr(),
                      gw.data_ptr(), xv[0], dim, xv[1], ov[1], dim, ctx.eps, _lib.dtype_code(x),
                      _lib.dtype_code(w), ws.data_ptr(), need, _lib.stream(x))
        return gx, gw.to(ctx.w_dtype), None


@compiler_disable
def fused_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(mean(x^2, -1) + eps) * weight, fp32 inside, x.dtype out."""
    _enabled(USE_FUSED_RMS_NORM, "fused_rms_norm")
    _lib.require_gpu("fused_rms_norm", x, weight)
    dim = x.shape[-1]
    if weight.shape != (dim,):
        raise ValueError(f"fused_rms_norm: weight shape {tuple(weight.shape)} != ({dim},)")
    return _RMSNormFunction.apply(x, weight, eps)


# ------------------------------------------------------- chunked cross-entropy
# fused_ops.py:1299-1577.  The token rows' softmax cross-entropy (and its
# gradient) run in hydra_ce_rows; the projections around it are plain GEMMs
# (hipBLASLt through F.linear / matmul).  Unlike the reference, the count of
# valid tokens stays on the device (no host synchronisation per chunk).
USE_CHUNKED_CROSS_ENTROPY = True
CROSS_ENTROPY_CHUNK_SIZE = 4096


def _ce_rows(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int,
             grad: torch.Tensor = None, grad_scale: torch.Tensor = None) -> torch.Tensor:
    """Per-row loss logsumexp(x) - x[t] (fp32, 0 for ignored rows) of a
    [rows, V] logits block with unit column stride; with `grad` (may be
    `logits` itself) also writes (softmax(x) - onehot(t)) * grad_scale[0]."""
    rows, V = logits.shape
    loss = torch.empty(rows, dtype=torch.float32, device=logits.device)
    _lib.call("hydra_ce_rows", logits.data_ptr(), rows, V, logits.stride(0), targets.data_ptr(),
              int(ignore_index), loss.data_ptr(), None, _lib.ptr(grad),
              grad.stride(0) if grad is not None else V, _lib.ptr(grad_scale),
              _lib.dtype_code(logits), _lib.stream(logits))
    return loss


class ChunkedCrossEntropyFunction(torch.autograd.Function):
    """fused_ops.py:1382-1531: mean token cross-entropy of hidden @ weight^T
    over tokens whose target is not ignore_index, computed chunk by chunk
    (logits of at most chunk_size tokens exist at a time); the backward
    recomputes each chunk's logits in fp32.  Out-of-range targets are
    handled as the reference does (:1407-1422): when any non-ignored target
    lies outside [0, vocab), the whole target vector -- ignore_index entries
    included -- is clamped into [0, vocab), and validity is taken from the
    clamped vector (so clamped ignore entries count).  The decision is made
    on the device (torch.where), without the reference's warning and its
    host synchronisation.  No valid token: loss 0 and zero gradients."""

    @staticmethod
    def forward(ctx, hidden_states, weight, targets, ignore_index, chunk_size):
        _lib.require_gpu("chunked_cross_entropy", hidden_states, weight, targets)
        dim = hidden_states.shape[-1]
        h = hidden_states.reshape(-1, dim)
        t = targets.reshape(-1).to(torch.int64)
        V = weight.shape[0]
        oob = ((t != ignore_index) & ((t < 0) | (t >= V))).any()
        t = torch.where(oob, t.clamp(0, V - 1), t).contiguous()
        total = torch.zeros((), dtype=torch.float32, device=h.device)
        for s in range(0, h.shape[0], chunk_size):
            logits = F.linear(h[s:s + chunk_size], weight).contiguous()
            total = total + _ce_rows(logits, t[s:s + chunk_size], ignore_index).sum()
        n_valid = (t != ignore_index).sum()
        ctx.save_for_backward(hidden_states, weight, t, n_valid)
        ctx.ignore_index, ctx.chunk_size = int(ignore_index), int(chunk_size)
        loss = torch.where(n_valid > 0, total / n_valid.clamp(min=1), torch.zeros_like(total))
        return loss.to(hidden_states.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        hidden_states, weight, t, n_valid = ctx.saved_tensors
        dim = hidden_states.shape[-1]
        h = hidden_states.reshape(-1, dim)
        wf = weight.float()
        scale = (grad_output.float() / n_valid.clamp(min=1)).reshape(1).contiguous()
        grad_h = torch.empty(h.shape, dtype=torch.float32, device=h.device)
        grad_w = torch.zeros(weight.shape, dtype=torch.float32, device=h.device)
        cs = ctx.chunk_size
        for s in range(0, h.shape[0], cs):
            hc = h[s:s + cs].float()
            g = F.linear(hc, wf).contiguous()  # logits, overwritten by their gradient
            _ce_rows(g, t[s:s + cs], ctx.ignore_index, grad=g, grad_scale=scale)
            grad_h[s:s + cs] = g @ wf
            grad_w += g.t() @ hc
        return (grad_h.view_as(hidden_states).to(hidden_states.dtype), grad_w.to(weight.dtype),
                None, None, None)


def chunked_cross_entropy(hidden_states: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                          ignore_index: int = -100, chunk_size: int = None) -> torch.Tensor:
    """fused_ops.py:1303-1379 (same value; the gradient runs through the HIP
    backward of ChunkedCrossEntropyFunction)."""
    return ChunkedCrossEntropyFunction.apply(hidden_states, weight, targets, ignore_index,
                                             chunk_size or CROSS_ENTROPY_CHUNK_SIZE)


def fused_chunked_cross_entropy(hidden_states: torch.Tensor, weight: torch.Tensor,
                                targets: torch.Tensor, ignore_index: int = -100,
                                chunk_size: int = None) -> torch.Tensor:
    """fused_ops.py:1534-1577 (its Liger branch does not apply: no Liger here)."""
    return chunked_cross_entropy(hidden_states, weight, targets, ignore_index, chunk_size)
