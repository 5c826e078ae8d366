"""CPU checks of the C ABI: the library loads, exports every entry point
include/hydra_amd.h declares (and the ctypes table covers them all), and
argument validation reports errors without touching a GPU."""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "hydra_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(hydra_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from hydra_amd import _lib

    lib_path = _lib.LIB_PATH
    assert lib_path.exists(), "build the library first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (hydra_\w+)", out))
    decl = declared_symbols()
    assert len(decl) >= 11
    missing = [s for s in decl if s not in exported]
    assert not missing, f"declared but not exported: {missing}"
    lib = _lib.load()
    for s in decl:
        assert getattr(lib, s) is not None
    # every compute entry point has a ctypes signature
    compute = [s for s in decl if s not in ("hydra_last_error", "hydra_abi_version")]
    assert sorted(_lib.SIGNATURES) == compute


def test_abi_version_and_error_path():
    from hydra_amd import _lib

    lib = _lib.load()
    assert lib.hydra_abi_version() == 111
    # dim = 0 is rejected before any HIP call
    rc = lib.hydra_rms_norm_fwd(None, None, None, 4, 0, 0, 0, ctypes.c_float(1e-6), 1, None)
    assert rc == _lib.ERR_ARG
    assert b"dim" in lib.hydra_last_error()
    with pytest.raises(ValueError, match="head_dim must be even"):
        _lib.call("hydra_rope_fwd", None, None, None, None, 1, 1, 1, 3,
                  (ctypes.c_int64 * 4)(3, 3, 3, 1), 1, 1, 0, None)
    with pytest.raises(ValueError, match="1 <= k <= L"):
        _lib.call("hydra_mod_topk", None, 1, 10, 10, 11, None, None, None, 0, 0, None)
    with pytest.raises(ValueError, match="1 <= L"):
        _lib.call("hydra_mod_topk", None, 1, 0, 16385, 1, None, None, None, 0, 0, None)
    with pytest.raises(ValueError, match="unknown score dtype"):
        _lib.call("hydra_mod_topk", None, 1, 16385, 16385, 5, None, None, None, 7, 0, None)
    with pytest.raises(ValueError, match="multiple of n_kv_heads"):
        st = (ctypes.c_int64 * 4)(0, 0, 0, 1)
        _lib.call("hydra_attn_fwd", None, None, None, None, None, None, 0, 1, 3, 2, 8, 16,
                  st, st, st, st, 1, ctypes.c_float(0.25), ctypes.c_float(0.0), None, 0, 1, None, 0, None)
    with pytest.raises(ValueError, match="mask mode needs key_mask"):
        st = (ctypes.c_int64 * 4)(0, 0, 0, 1)
        _lib.call("hydra_attn_fwd", None, None, None, None, None, None, 1, 1, 2, 2, 8, 16,
                  st, st, st, st, 1, ctypes.c_float(0.25), ctypes.c_float(0.0), None, 0, 1, None, 0, None)
    with pytest.raises(ValueError, match="unknown flag"):
        _lib.call("hydra_ccgqa_prep_fwd", None, 48, None, None, None, None, None, None, None, 0,
                  None, None, None, 1, 4, 2, 1, 16, 3, 128, 1, None)
    # the tiled conv-weight layout is offered for bf16 MFMA head dims only
    # (a layout small enough for the 64 KB LDS assumed without a device)
    assert _lib.query("hydra_ccgqa_prep_tiled_ok", 4, 1, 32, _lib.BF16) == 1
    assert _lib.query("hydra_ccgqa_prep_tiled_ok", 4, 1, 32, _lib.F32) == 0
    assert _lib.query("hydra_ccgqa_prep_tiled_ok", 4, 1, 48, _lib.BF16) == 0
    assert _lib.query("hydra_ccgqa_prep_tiled_ok", 4, 3, 64, _lib.BF16) == 0
    # empty work is a no-op success
    _lib.call("hydra_swiglu_fwd", None, None, None, 0, 8, 8, 8, 8, 1, None)
    _lib.call("hydra_stream_copy", None, None, 0, None)
    with pytest.raises(ValueError, match="multiple of 16"):
        _lib.call("hydra_stream_copy", 16, 32, 24, None)
    with pytest.raises(ValueError, match="16-byte aligned"):
        _lib.call("hydra_stream_copy", 8, 32, 32, None)
