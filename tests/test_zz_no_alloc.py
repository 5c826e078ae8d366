"""The allocation-free RMSNorm backward (hydra_rms_norm_bwd_noalloc), called
through the C ABI: two calls in a row (the second smaller, so leftovers of
the first in the fixed scratch would show) give the same bits as the
allocating hydra_rms_norm_bwd, and both match the oracle; a dim beyond the
scratch's maximum is rejected with an error."""
from __future__ import annotations

import pytest
import torch

from conftest import max_rel_err
from oracle import fused_ops as ofo

pytestmark = pytest.mark.gpu


def _bwd(name, x, w, gy):
    from hydra_amd import _lib

    rows, dim = x.shape
    gx = torch.empty_like(x)
    gw = torch.empty_like(w)
    args = (x.data_ptr(), w.data_ptr(), gy.data_ptr(), gx.data_ptr(), gw.data_ptr(), rows, dim,
            dim, dim, dim, 1e-6, _lib.dtype_code(x), _lib.dtype_code(w))
    if name == "hydra_rms_norm_bwd":  # the allocating form takes torch-provided scratch
        need = _lib.query("hydra_rms_norm_bwd_workspace", rows, dim)
        ws = _lib.scratch(need, x)
        _lib.call(name, *args, ws.data_ptr(), need, _lib.stream(x))
    else:
        _lib.call(name, *args, _lib.stream(x))
    return gx, gw


@pytest.mark.parametrize("dtype,wdtype", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                          (torch.bfloat16, torch.float32)])
def test_noalloc_matches_allocating_entry_point(cuda, dtype, wdtype):
    g = torch.Generator().manual_seed(31)
    for rows, dim in ((16384, 768), (1000, 512), (37, 100)):  # each call smaller than the last
        x = torch.randn(rows, dim, generator=g).to(dtype).to(cuda)
        gy = torch.randn(rows, dim, generator=g).to(dtype).to(cuda)
        w = (1 + 0.1 * torch.randn(dim, generator=g)).to(wdtype).to(cuda)
        gx_n, gw_n = _bwd("hydra_rms_norm_bwd_noalloc", x, w, gy)
        gx_a, gw_a = _bwd("hydra_rms_norm_bwd", x, w, gy)
        torch.cuda.synchronize()
        assert torch.equal(gx_n, gx_a) and torch.equal(gw_n, gw_a), (rows, dim)
        gx_r, gw_r = ofo.rms_norm_backward(x.cpu().float(), w.cpu().float(), gy.cpu().float(), 1e-6)
        tol = 1e-5 if dtype == torch.float32 else 2e-2
        assert max_rel_err(gx_n.cpu(), gx_r) < tol
        assert max_rel_err(gw_n.cpu(), gw_r) < (1e-5 if wdtype == torch.float32 else 2e-2)


def test_noalloc_rejects_dim_beyond_scratch(cuda):
    x = torch.randn(4, 4104, device=cuda)
    w = torch.ones(4104, device=cuda)
    with pytest.raises(ValueError, match="maximum"):
        _bwd("hydra_rms_norm_bwd_noalloc", x, w, x)
