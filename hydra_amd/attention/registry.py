"""Backend registry (hydra/attention/registry.py:7-49): only CCGQA, under the
names "ccqa" and "ccgqa"; anything else is a ValueError."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional


@dataclass(frozen=True, slots=True)
class HybridAttentionBackend:
    """Resolved hybrid-attention backend (registry.py:7-14)."""

    name: str


def is_hybrid_attention_backend_available(name: str) -> bool:
    """registry.py:17-20."""
    return str(name).strip().lower() in ("ccqa", "ccgqa")


def available_hybrid_attention_backends() -> tuple[str, ...]:
    """registry.py:23-25."""
    return ("ccqa",)


def resolve_hybrid_attention_backend(requested: Optional[str], *,
                                     default: str = "ccqa") -> HybridAttentionBackend:
    """registry.py:28-49: None -> ccqa; "ccqa"/"ccgqa" -> ccqa; else ValueError."""
    if requested is None:
        return HybridAttentionBackend("ccqa")
    req = str(requested).strip().lower()
    if req in ("ccqa", "ccgqa"):
        return HybridAttentionBackend("ccqa")
    raise ValueError(f"Unknown attention backend '{requested}'. Only 'ccgqa' is supported.")
