"""CCGQA kernels (hydra/attention/backends/ccgqa/kernels/__init__.py)."""
from .fused_attention import ccgqa_attention_fused

__all__ = ["ccgqa_attention_fused"]
