"""Loading the reference's training checkpoints into the hot-path modules.

The reference writes one dict per checkpoint (hydra/training/checkpointing.py:
134-150): {"step", "model": model.state_dict(), "optimizer", "scaler",
"config", "rng_state", "metrics", ...}, with the model unwrapped from
torch.compile first (:131-132).  The hot-path modules here keep the
reference's parameter names (CCGQAAttention also migrates its legacy keys,
attention.py:333-383), so a submodule's state is the "model" entries under
that submodule's prefix.  Files are read with torch.load(weights_only=True)
only: nothing in a checkpoint is executed."""
from __future__ import annotations

from pathlib import Path
from typing import Mapping, Union

import torch

_COMPILE_PREFIX = "_orig_mod."


def _numpy_rng_globals() -> list:
    """The numpy types a reference checkpoint's rng_state["numpy"]
    (np.random.get_state(), checkpointing.py:17-33) pickles: ndarray
    reconstruction, dtype and the uint32 dtype class.  Allow-listing them
    keeps the load weights-only: these rebuild arrays, they run no code."""
    import numpy as np

    try:
        from numpy._core.multiarray import _reconstruct
    except ImportError:  # numpy < 2
        from numpy.core.multiarray import _reconstruct
    return [_reconstruct, np.ndarray, np.dtype, type(np.dtype(np.uint32))]


def read_checkpoint(path: Union[str, Path]) -> dict:
    """The checkpoint dict, loaded on the CPU with weights_only=True and
    numpy's array types allow-listed (the reference stores numpy's RNG state
    in every checkpoint).  A file the safe loader still refuses raises,
    naming the file; pass its "model" dict to `module_state` instead."""
    try:
        with torch.serialization.safe_globals(_numpy_rng_globals()):
            return torch.load(str(path), map_location="cpu", weights_only=True)
    except Exception as e:  # the safe unpickler's refusal, or a bad file
        raise RuntimeError(f"read_checkpoint: {path} cannot be read with weights_only=True ({e})") from e


def module_state(checkpoint: Mapping, prefix: str) -> dict:
    """The entries of checkpoint["model"] (or of `checkpoint` itself when it
    is already a state_dict) under `prefix` (e.g. "blocks.3.attention."),
    with the prefix and any torch.compile "_orig_mod." segments removed."""
    sd = checkpoint.get("model", checkpoint) if isinstance(checkpoint, Mapping) else checkpoint
    if not isinstance(sd, Mapping):
        raise TypeError("module_state: checkpoint['model'] is not a state_dict")
    out = {}
    for key, val in sd.items():
        k = key.replace(_COMPILE_PREFIX, "")
        if prefix and not k.startswith(prefix):
            continue
        out[k[len(prefix):]] = val
    if not out:
        raise KeyError(f"module_state: no entries under prefix {prefix!r}")
    return out


def load_module_from_checkpoint(module: torch.nn.Module, checkpoint: Union[str, Path, Mapping],
                                prefix: str = "", strict: bool = True):
    """Loads one hot-path module (CCGQAAttention, RMSNorm, SwiGLUMLPFused,
    MoDRouter, ...) from a reference checkpoint file or dict; returns
    load_state_dict's (missing, unexpected) keys."""
    ckpt = read_checkpoint(checkpoint) if isinstance(checkpoint, (str, Path)) else checkpoint
    return module.load_state_dict(module_state(ckpt, prefix), strict=strict)
