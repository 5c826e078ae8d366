"""hydra_amd.attention -- the surface of hydra/attention/__init__.py."""

from .registry import (
    HybridAttentionBackend,
    available_hybrid_attention_backends,
    is_hybrid_attention_backend_available,
    resolve_hybrid_attention_backend,
)
from .backends.ccgqa.attention import CCGQAAttention
from .factory import build_hybrid_attention_module

__all__ = [
    "HybridAttentionBackend",
    "available_hybrid_attention_backends",
    "is_hybrid_attention_backend_available",
    "resolve_hybrid_attention_backend",
    "CCGQAAttention",
    "build_hybrid_attention_module",
]
