"""CCGQA backend bundle (hydra/attention/backends/ccgqa/__init__.py:12-15):
the package stays import-light; `build_ccqa_attention` is backend.py's,
imported when first called."""
from __future__ import annotations

from typing import Any


def build_ccqa_attention(**kwargs: Any):
    """Standard constructor for the CCQA backend (backend.py:8-17)."""
    from .backend import build_ccqa_attention as _build

    return _build(**kwargs)


__all__ = ["build_ccqa_attention"]
