"""pytest configuration: markers, GPU gating, shared helpers."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def max_rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """Normwise max relative error: max|a - b| / max|b| (both in fp64).

    This is the metric the tolerances (1e-5 fp32, 2e-2 bf16) are stated in;
    elementwise relative error is ill-conditioned near zero."""
    a64, b64 = a.detach().double().cpu(), b.detach().double().cpu()
    den = b64.abs().max().item()
    num = (a64 - b64).abs().max().item()
    return num / den if den > 0 else num


def bf16_from_bits(arr) -> torch.Tensor:
    """uint16 bf16 bit patterns (as stored in the golden .npz) -> fp32 tensor."""
    import numpy as np

    a = np.asarray(arr).astype(np.uint32) << 16
    return torch.from_numpy(a.view(np.float32).copy())


@pytest.fixture(scope="session")
def cuda():
    return torch.device("cuda:0")
