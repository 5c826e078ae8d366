"""CCGQA backend bundle (hydra/attention/backends/ccgqa/__init__.py:12-15)."""
from __future__ import annotations

from typing import Any


def build_ccqa_attention(**kwargs: Any):
    """Standard constructor for the CCQA backend (backend.py:8-17)."""
    from .attention import CCGQAAttention

    return CCGQAAttention(**kwargs)


__all__ = ["build_ccqa_attention"]
