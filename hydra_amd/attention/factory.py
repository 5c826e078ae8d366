"""Attention module factory (hydra/attention/factory.py:28-89)."""
from __future__ import annotations

import os
from typing import Any, TypedDict

import torch.nn as nn


class CCGQAKwargs(TypedDict, total=False):
    use_rope: bool
    use_qk_norm: bool
    use_convs: bool
    use_qk_mean: bool
    use_value_shift: bool
    conv_kernel_size: int
    use_fused_kernel: bool


_ALLOWED = {"use_rope", "use_qk_norm", "use_convs", "use_qk_mean", "use_value_shift",
            "conv_kernel_size", "use_fused_kernel"}


def build_hybrid_attention_module(requested: str, *, dim: int, n_heads: int, n_kv_heads: int,
                                  max_seq_len: int, compression_factor: int,
                                  attention_kwargs: dict[str, Any] | CCGQAKwargs) -> nn.Module:
    """Instantiate the CCGQA module; unknown backend names raise ValueError,
    kwargs outside the whitelist are dropped (factory.py:65-74), and
    HYDRA_CCQA_USE_FUSED_KERNEL overrides use_fused_kernel (factory.py:76-80)."""
    req = str(requested).strip().lower()
    if req not in ("ccqa", "ccgqa"):
        raise ValueError(f"Unknown attention backend '{requested}'. Only 'ccgqa' is supported.")
    from .backends.ccgqa.attention import CCGQAAttention

    kw = {k: v for k, v in attention_kwargs.items() if k in _ALLOWED}
    env = os.environ.get("HYDRA_CCQA_USE_FUSED_KERNEL", "").strip().lower()
    if env in {"1", "true", "yes", "y"}:
        kw["use_fused_kernel"] = True
    elif env in {"0", "false", "no", "n"}:
        kw["use_fused_kernel"] = False
    return CCGQAAttention(dim=dim, n_heads=n_heads, n_kv_heads=n_kv_heads,
                          compression_factor=compression_factor, max_seq_len=max_seq_len, **kw)
