"""ctypes binding of libhydra_amd.so (the C ABI declared in include/hydra_amd.h).

The library is loaded after torch, so it binds to the HIP runtime torch already
has in the process.  Tensors cross the boundary as raw device pointers, sizes,
element strides and torch's current HIP stream; no torch type crosses it.

There is no fallback: if the library is missing, or a tensor is not on a GPU,
the call raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("HYDRA_AMD_LIB", Path(__file__).with_name("libhydra_amd.so")))

# status / dtype / flag codes (include/hydra_amd.h)
OK, ERR_ARG, ERR_LAUNCH, ERR_UNSUPPORTED = 0, 1, 2, 3
F32, BF16, F16 = 0, 1, 2
CCGQA_CONVS, CCGQA_QK_MEAN, CCGQA_VALUE_SHIFT, CCGQA_QK_NORM, CCGQA_ROPE = 1, 2, 4, 8, 16
CCGQA_V_TRANSPOSED = 32
CCGQA_W_TILED = 64
MASK_NONE, MASK_KEY_PADDING, MASK_REFERENCE_SDPA = 0, 1, 2
SCATTER_ADD, SCATTER_REPLACE, SCATTER_ADD_SEQ = 0, 1, 2
NORM_NONE, NORM_RMS, NORM_ADA = 0, 1, 2
LINEAR_W_TILED = 1

_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_I64P = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes, in declaration order of include/hydra_amd.h
SIGNATURES = {
    "hydra_rms_norm_fwd": [_P, _P, _P, _I64, _I64, _I64, _I64, _F, _I, _P],
    "hydra_rope_fwd": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64P, _I64, _I, _I, _P],
    "hydra_swiglu_fwd": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "hydra_qk_norm_fwd": [_P, _P, _P, _P, _I64, _I64, _I64, _F, _F, _I, _P],
    "hydra_rms_norm_bwd": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _P, _I64, _P],
    "hydra_rms_norm_bwd_workspace": [_I64, _I64],
    "hydra_rms_norm_bwd_noalloc": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _P],
    "hydra_rope_bwd": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64P, _I64, _I, _I, _P],
    "hydra_swiglu_bwd": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "hydra_qk_norm_bwd": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _F, _I, _P],
    "hydra_ccgqa_prep_fwd": [_P, _I64, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P,
                             _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _P],
    "hydra_attn_fwd": [_P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64,
                       _I64P, _I64P, _I64P, _I64P, _I, _F, _F, _P, _I, _I, _P, _I64, _P],
    "hydra_attn_fwd_workspace": [_I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _I64P, _I64P, _I, _I, _I,
                                 _I64P],
    "hydra_attn_bwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                       _I64P, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P, _P, _I, _I, _F, _I, _P,
                       _I64, _P],
    "hydra_attn_bwd_workspace": [_I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P,
                                 _I64P, _I64P, _I, _I, _I, _I64P],
    "hydra_linear_fwd": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I, _I, _P],
    "hydra_ce_rows": [_P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _P, _I, _P],
    "hydra_ccgqa_prep_tiled_ok": [_I64, _I64, _I64, _I],
    "hydra_ccgqa_prep_faults": [_P],
    "hydra_ccgqa_prep_bwd": [_P, _I64, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _P,
                             _I64, _I64, _I64, _I64, _I64, _I, _I, _P],
    "hydra_causal_im2col": [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "hydra_causal_col2im": [_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _P],
    "hydra_embedding_fwd": [_P, _I64, _P, _I64, _I64, _I64, _F, _P, _I64, _I, _P],
    "hydra_residual_norm_fwd": [_P, _I64, _P, _I64, _F, _P, _P, _P, _F, _I, _P, _I64, _P, _I64,
                                _I64, _I64, _I, _I, _P],
    "hydra_mor_update": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I, _P],
    "hydra_mor_route": [_P, _I64, _P, _P, _P, _I64, _I64, _I, _P],
    "hydra_mod_topk": [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _I, _I, _P],
    "hydra_mod_gather": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "hydra_mod_scatter": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _P],
    "hydra_stream_copy": [_P, _P, _I64, _P],
    "hydra_clock_probe": [_P, _I, _I, _I64P, _P],
    "hydra_attn_clock_stamps": [_P, _I64],
}

# entry points that return a value (not a status) of type int64_t
_RETURNS_INT64 = {"hydra_rms_norm_bwd_workspace"}

_lib = None


class HydraError(RuntimeError):
    """A C-ABI call returned a nonzero status."""


def load() -> ctypes.CDLL:
    """Load (once) and return the shared library; raise if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"hydra_amd: {LIB_PATH} is not built; run "
                "`python -c 'import __graft_entry__ as g; g.build()'` (needs hipcc)")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.hydra_last_error.restype = ctypes.c_char_p
        lib.hydra_last_error.argtypes = []
        lib.hydra_abi_version.restype = ctypes.c_int
        lib.hydra_abi_version.argtypes = []
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int64 if name in _RETURNS_INT64 else ctypes.c_int
        _lib = lib
    return _lib


def available() -> bool:
    """True when the library is built and loads."""
    try:
        load()
        return True
    except (OSError, RuntimeError):
        return False


def call(name: str, *args) -> None:
    """Call an entry point and raise HydraError (ValueError for bad
    arguments) on a nonzero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != OK:
        msg = lib.hydra_last_error().decode(errors="replace")
        if rc == ERR_ARG:
            raise ValueError(f"{name}: {msg}")
        raise HydraError(f"{name} failed ({rc}): {msg}")


def call_status(name: str, *args) -> int:
    """Call an entry point and return its status (for callers that handle
    HYDRA_ERR_UNSUPPORTED themselves); check() raises for the others."""
    return int(getattr(load(), name)(*args))


def check(rc: int, name: str) -> None:
    if rc != OK:
        msg = load().hydra_last_error().decode(errors="replace")
        if rc == ERR_ARG:
            raise ValueError(f"{name}: {msg}")
        raise HydraError(f"{name} failed ({rc}): {msg}")


def prep_faults() -> int:
    """hydra_ccgqa_prep_faults: prep tiles (on the current device, since
    load) whose epilogue timed out waiting for the QK-mean terms; 0 on a
    working device."""
    n = ctypes.c_uint(0)
    call("hydra_ccgqa_prep_faults", ctypes.byref(n))
    return int(n.value)


def scratch(nbytes: int, like: torch.Tensor) -> torch.Tensor:
    """Device scratch of nbytes from torch's caching allocator on like's
    device (the library owns no memory between calls)."""
    return torch.empty(max(int(nbytes), 0), dtype=torch.uint8, device=like.device)


def query(name: str, *args) -> int:
    """Call an entry point that returns a value rather than a status."""
    return int(getattr(load(), name)(*args))


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"hydra_amd: unsupported dtype {t.dtype}") from None


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def strides(t: torch.Tensor):
    arr = (ctypes.c_int64 * t.dim())(*t.stride())
    return arr


def stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(name: str, *tensors) -> None:
    """The product runs on the GPU only: a CPU tensor is an error, never a
    reason to fall back."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"{name}: hydra_amd runs its HIP kernels on GPU tensors only "
                f"(got a tensor on {t.device})")
    dev = None
    for t in tensors:
        if t is not None:
            if dev is None:
                dev = t.device
            elif t.device != dev:
                raise RuntimeError(f"{name}: tensors on different devices ({dev}, {t.device})")
