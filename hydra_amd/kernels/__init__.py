"""hydra_amd.kernels -- the fused-op surface of hydra/kernels/__init__.py
(:13-37, :140-192) backed by the gfx950 HIP library."""

from .fused_ops import (
    CROSS_ENTROPY_CHUNK_SIZE,
    USE_CHUNKED_CROSS_ENTROPY,
    ChunkedCrossEntropyFunction,
    chunked_cross_entropy,
    fused_chunked_cross_entropy,
    HIP_AVAILABLE,
    TRITON_AVAILABLE,
    USE_FUSED_QK_NORM,
    USE_FUSED_RMS_NORM,
    USE_FUSED_ROPE,
    USE_FUSED_SWIGLU,
    USE_TRITON_KERNELS,
    fused_qk_norm,
    fused_rms_norm,
    fused_rope,
    fused_swiglu,
    get_kernel_status,
    set_use_triton_kernels,
)

__all__ = [
    "chunked_cross_entropy",
    "fused_chunked_cross_entropy",
    "ChunkedCrossEntropyFunction",
    "CROSS_ENTROPY_CHUNK_SIZE",
    "USE_CHUNKED_CROSS_ENTROPY",
    "fused_rope",
    "fused_qk_norm",
    "fused_swiglu",
    "fused_rms_norm",
    "TRITON_AVAILABLE",
    "HIP_AVAILABLE",
    "USE_TRITON_KERNELS",
    "USE_FUSED_ROPE",
    "USE_FUSED_QK_NORM",
    "USE_FUSED_SWIGLU",
    "USE_FUSED_RMS_NORM",
    "set_use_triton_kernels",
    "get_kernel_status",
]
