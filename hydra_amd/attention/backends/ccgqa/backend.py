"""hydra/attention/backends/ccgqa/backend.py:8-17."""
from __future__ import annotations

from typing import Any

from .attention import CCGQAAttention


def build_ccqa_attention(**kwargs: Any) -> CCGQAAttention:
    return CCGQAAttention(**kwargs)
