"""Fused RMSNorm / RoPE / SwiGLU / QK-norm on MI355X.

Drop-in for hydra/kernels/fused_ops.py: same function names, signatures,
flags and error behaviour; the Triton kernels are replaced by the gfx950 HIP
kernels of libhydra_amd.so.  The flag names keep the reference's
"TRITON" spelling so callers need no change; here they mean "the HIP
library is loaded".

Forward only.  The ops are wrapped in autograd Functions whose backward
raises, so a training graph fails loudly instead of getting no gradient.
"""
from __future__ import annotations

import os
from typing import Tuple

import torch

from .. import _lib
from .._autograd import track

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
# Backward kernels are not part of this build.
USE_FUSED_SWIGLU_BACKWARD = False
USE_FUSED_RMS_NORM_BACKWARD = False
USE_FUSED_QK_NORM_BACKWARD = False
LIGER_CE_AVAILABLE = False
USE_LIGER_CE = False


def set_use_triton_kernels(enabled: bool) -> None:
    """Enable or disable the fused kernels globally (fused_ops.py:121-146).

    Raises RuntimeError when enabling without the HIP library, as the
    reference does without Triton.  While disabled, the fused_* functions
    raise instead of running: this build has no non-HIP path."""
    global USE_TRITON_KERNELS, USE_FUSED_ROPE, USE_FUSED_QK_NORM, USE_FUSED_SWIGLU, USE_FUSED_RMS_NORM
    if enabled and not TRITON_AVAILABLE:
        raise RuntimeError("hydra_amd HIP library is not available (build it with __graft_entry__.build())")
    USE_TRITON_KERNELS = bool(enabled)
    USE_FUSED_ROPE = USE_TRITON_KERNELS and _env_on("HYDRA_ENABLE_FUSED_ROPE", "1") and not _env_on("HYDRA_DISABLE_FUSED_ROPE", "0")
    USE_FUSED_QK_NORM = USE_TRITON_KERNELS
    USE_FUSED_SWIGLU = USE_TRITON_KERNELS
    USE_FUSED_RMS_NORM = USE_TRITON_KERNELS and _env_on("HYDRA_ENABLE_FUSED_RMS_NORM", "1") and not _env_on("HYDRA_DISABLE_FUSED_RMS_NORM", "0")


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


_track = track


# ---------------------------------------------------------------------------
# 1. RoPE (fused_ops.py:240-297)
# ---------------------------------------------------------------------------
@compiler_disable
def fused_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotary embedding on interleaved pairs.

    x: [B, n_heads, S, head_dim] (any strides); cos/sin: [1, 1, Smax, hd/2]
    or [S, hd/2].  Returns a contiguous tensor of x's shape and dtype."""
    _enabled(USE_FUSED_ROPE, "fused_rope")
    _lib.require_gpu("fused_rope", x, cos, sin)
    B, H, S, D = x.shape
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
    out = torch.empty((B, H, S, D), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("hydra_rope_fwd", x.data_ptr(), cos.data_ptr(), sin.data_ptr(), out.data_ptr(),
                  B, H, S, D, _lib.strides(x), cos.stride(0), _lib.dtype_code(x),
                  _lib.dtype_code(cos), _lib.stream(x))
    return _track(out, x)


# ---------------------------------------------------------------------------
# 2. QK-norm (fused_ops.py:474-526)
# ---------------------------------------------------------------------------
@compiler_disable
def fused_qk_norm(q: torch.Tensor, k: torch.Tensor, scale: float,
                  temperature: float = 1.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """q * rsqrt(sum q^2 + 1e-8) * scale and k * rsqrt(sum k^2 + 1e-8) *
    scale * temperature over the last dim."""
    _enabled(USE_FUSED_QK_NORM, "fused_qk_norm")
    _lib.require_gpu("fused_qk_norm", q, k)
    if q.dtype != k.dtype or q.shape[-1] != k.shape[-1]:
        raise ValueError("fused_qk_norm: q and k must share dtype and head_dim")
    qc, kc = q.contiguous(), k.contiguous()
    qo, ko = torch.empty_like(qc), torch.empty_like(kc)
    hd = q.shape[-1]
    with torch.cuda.device(q.device):
        _lib.call("hydra_qk_norm_fwd", qc.data_ptr(), kc.data_ptr(), qo.data_ptr(), ko.data_ptr(),
                  qc.numel() // hd, kc.numel() // hd, hd, float(scale), float(temperature),
                  _lib.dtype_code(q), _lib.stream(q))
    return _track(qo, q, k), _track(ko, q, k)


# ---------------------------------------------------------------------------
# 3. SwiGLU (fused_ops.py:808-843)
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


@compiler_disable
def fused_swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up.  gate/up may be the strided halves of one gate_up
    tensor; they are read in place (no contiguous copies)."""
    _enabled(USE_FUSED_SWIGLU, "fused_swiglu")
    _lib.require_gpu("fused_swiglu", gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("fused_swiglu: gate and up must have the same shape and dtype")
    gv, uv = _rows_view(gate), _rows_view(up)
    if gv is None:
        gate = gate.contiguous()
        gv = _rows_view(gate)
    if uv is None:
        up = up.contiguous()
        uv = _rows_view(up)
    hidden = gate.shape[-1] if gate.dim() else 1
    out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    with torch.cuda.device(gate.device):
        _lib.call("hydra_swiglu_fwd", gate.data_ptr(), up.data_ptr(), out.data_ptr(),
                  gv[0], hidden, gv[1], uv[1], hidden, _lib.dtype_code(gate), _lib.stream(gate))
    return _track(out, gate, up)


# ---------------------------------------------------------------------------
# 4. RMSNorm (fused_ops.py:1114-1159)
# ---------------------------------------------------------------------------
@compiler_disable
def fused_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(mean(x^2, -1) + eps) * weight, fp32 inside, x.dtype out."""
    _enabled(USE_FUSED_RMS_NORM, "fused_rms_norm")
    _lib.require_gpu("fused_rms_norm", x, weight)
    dim = x.shape[-1]
    if weight.shape != (dim,):
        raise ValueError(f"fused_rms_norm: weight shape {tuple(weight.shape)} != ({dim},)")
    w = weight if weight.dtype == x.dtype else weight.to(x.dtype)
    w = w.contiguous()
    xv = _rows_view(x)
    if xv is None:
        x = x.contiguous()
        xv = _rows_view(x)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("hydra_rms_norm_fwd", x.data_ptr(), w.data_ptr(), out.data_ptr(),
                  xv[0], dim, xv[1], dim, float(eps), _lib.dtype_code(x), _lib.stream(x))
    return _track(out, x, weight)
