"""The CCQA backend's constructor (hydra/attention/backends/ccgqa/backend.py:8-17):
the registry and the factory select the backend by name; this builds the
module itself."""
from __future__ import annotations

from typing import Any

from .attention import CCGQAAttention


def build_ccqa_attention(**kwargs: Any) -> CCGQAAttention:
    """CCGQAAttention(**kwargs) -- the gfx950 module with the reference's
    constructor arguments."""
    return CCGQAAttention(**kwargs)
