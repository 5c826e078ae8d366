"""GPU parity of Mixture-of-Depths hard routing: top-k indices bit-exact
(value-descending with lowest-index ties, and ascending), mask exact,
torch.topk's value sequence reproduced, row gather and residual scatter
bit-exact against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN, bf16_from_bits
from oracle import mod as omod

pytestmark = pytest.mark.gpu


def _check_topk(scores: torch.Tensor, k: int, cuda, mask_dtype=torch.float32):
    from hydra_amd.routing import mod_topk

    desc, srt, mask = mod_topk(scores.to(cuda), k, mask_dtype=mask_dtype)
    want = omod.topk_desc_lowest_index(scores.float().numpy(), k)
    assert np.array_equal(desc.cpu().numpy(), want)
    assert np.array_equal(srt.cpu().numpy(), omod.sorted_indices(want))
    assert np.array_equal(mask.float().cpu().numpy(), omod.mask_from_indices(want, scores.shape[1]))
    vals = torch.topk(scores.float(), k, dim=-1).values
    got_vals = torch.gather(scores.float(), 1, desc.cpu())
    assert torch.equal(torch.nan_to_num(got_vals, nan=1e30), torch.nan_to_num(vals, nan=1e30))


def test_topk_c4(cuda):
    """Config 4: fp32 logits [8, 4096] with 5% duplicated entries, k = 3072."""
    g = torch.Generator().manual_seed(0)
    s = omod.make_tied_logits(8, 4096, 0.05, g)
    _check_topk(s, omod.router_k(4096, 0.75), cuda)


@pytest.mark.parametrize("B,L,k", [(1, 1, 1), (3, 64, 1), (3, 64, 64), (2, 1000, 999),
                                   (2, 16384, 12288), (5, 333, 100), (70, 128, 96)])
def test_topk_sizes(cuda, B, L, k):
    g = torch.Generator().manual_seed(L + k)
    _check_topk(omod.make_tied_logits(B, L, 0.05, g), k, cuda)


def test_topk_special_values(cuda):
    row = torch.tensor([[1.0, 3.0, 3.0, -1.0, 3.0, 0.5, 0.0, -0.0, float("nan"), float("inf"),
                         float("-inf"), -0.0, float("nan"), 0.0, 2.0, 2.0]])
    for k in (1, 3, 8, 16):
        from hydra_amd.routing import mod_topk

        desc, _, _ = mod_topk(row.to(cuda), k)
        assert np.array_equal(desc.cpu().numpy(), omod.topk_desc_lowest_index(row.numpy(), k))


def test_topk_bf16_scores_and_mask(cuda):
    g = torch.Generator().manual_seed(3)
    s = torch.randn(4, 2048, generator=g).to(torch.bfloat16)  # bf16 scores tie often
    _check_topk(s, 1536, cuda, mask_dtype=torch.bfloat16)


@pytest.mark.parametrize("cap", ["0750", "0500", "0125"])
def test_router_golden_scores(cuda, cap):
    """Golden router scores (written by running MoDRouter): our indices are
    the lowest-index-tie order of the same value sequence torch.topk gave."""
    from hydra_amd.routing import mod_topk

    d = np.load(GOLDEN / f"mod_router_cap{cap}.npz")
    s = torch.from_numpy(d["scores"])
    k = d["indices"].shape[1]
    desc, _, mask = mod_topk(s.to(cuda), k, mask_dtype=torch.float32)
    assert np.array_equal(desc.cpu().numpy(), d["stable_order"])
    assert np.array_equal(np.take_along_axis(d["scores"], desc.cpu().numpy(), 1),
                          np.take_along_axis(d["scores"], d["indices"], 1))


def test_router_module(cuda):
    from hydra_amd.routing import MoDRouter

    d = np.load(GOLDEN / "mod_router_cap0750.npz")
    r = MoDRouter(dim=64, capacity_ratio=0.75)
    with torch.no_grad():
        r.router.weight.copy_(bf16_from_bits(d["w"]))
        r.router.bias.copy_(bf16_from_bits(d["b"]))
    r = r.to(cuda).eval()
    x = bf16_from_bits(d["x"]).to(cuda)
    with torch.no_grad():
        mask, idx, scores = r(x, return_scores=True)
    want = omod.topk_desc_lowest_index(scores.cpu().numpy(), d["indices"].shape[1])
    assert np.array_equal(idx.cpu().numpy(), want)
    assert np.array_equal(mask.cpu().numpy(), omod.mask_from_indices(want, x.shape[1]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gather_scatter_c4(cuda, dtype):
    """Config 4 rows: x [8,4096,1280], y [8,3072,1280]."""
    from hydra_amd.routing import gather_by_indices, weighted_residual_scatter

    g = torch.Generator().manual_seed(5)
    s = omod.make_tied_logits(8, 4096, 0.05, g)
    idx = torch.from_numpy(omod.sorted_indices(omod.topk_desc_lowest_index(s.numpy(), 3072)))
    x = torch.randn(8, 4096, 1280, generator=g).to(dtype)
    y = torch.randn(8, 3072, 1280, generator=g).to(dtype)
    xs = gather_by_indices(x.to(cuda), idx.to(cuda)).cpu()
    assert torch.equal(xs, omod.gather(x, idx))
    h = x.to(cuda)
    weighted_residual_scatter(h, y.to(cuda), idx.to(cuda))
    assert torch.equal(h.cpu(), omod.residual_scatter(x, y, idx))


def test_weighted_and_replace_scatter(cuda):
    from hydra_amd.routing import scatter_replace, weighted_residual_scatter

    g = torch.Generator().manual_seed(6)
    x = torch.randn(3, 100, 48, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(100, generator=g)[:30] for _ in range(3)])
    y = torch.randn(3, 30, 48, generator=g).to(torch.bfloat16)
    w = torch.rand(3, 30, generator=g)
    h = x.to(cuda)
    weighted_residual_scatter(h, y.to(cuda), idx.to(cuda), w.to(cuda))
    assert torch.equal(h.cpu(), omod.residual_scatter(x, y, idx, w))
    r = x.to(cuda)
    scatter_replace(r, y.to(cuda), idx.to(cuda))
    assert torch.equal(r.cpu(), omod.replace_scatter(x, y, idx))


def test_odd_width_rows_scalar_path(cuda):
    from hydra_amd.routing import gather_by_indices, scatter_add_by_indices

    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 50, 13, generator=g)
    idx = torch.stack([torch.randperm(50, generator=g)[:20] for _ in range(2)])
    assert torch.equal(gather_by_indices(x.to(cuda), idx.to(cuda)).cpu(), omod.gather(x, idx))
    y = torch.randn(2, 20, 13, generator=g)
    h = x.to(cuda)
    scatter_add_by_indices(h, y.to(cuda), idx.to(cuda))
    assert torch.equal(h.cpu(), omod.residual_scatter(x, y, idx))


def test_mod_mlp_hard_path(cuda):
    """MoDMLPWrapper._forward_hard and the fused residual form against the
    oracle composition (blocks.py:243-269, :603)."""
    from hydra_amd.layers import SwiGLUMLPFused
    from hydra_amd.routing import MoDMLPWrapper
    from oracle import fused_ops as ofo

    g = torch.Generator().manual_seed(8)
    D, Hd = 64, 96
    mlp = SwiGLUMLPFused(D, Hd)
    wrap = MoDMLPWrapper(mlp, D, capacity_ratio=0.75, warmup_steps=0)
    with torch.no_grad():
        for p in wrap.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.05)
    wrap.set_global_step(1)
    wrap = wrap.to(cuda).eval()
    x = torch.randn(2, 128, D, generator=g)
    h = torch.randn(2, 128, D, generator=g)
    with torch.no_grad():
        out = wrap(x.to(cuda)).cpu()
        hr = wrap.forward_residual(h.to(cuda), x.to(cuda)).cpu()
    with torch.no_grad():  # the routing decision is taken on the device's scores
        scores = wrap.mod_router.forward_logits(x.to(cuda)).cpu()
    idx = torch.from_numpy(omod.sorted_indices(omod.topk_desc_lowest_index(scores.numpy(), 96)))
    xs = omod.gather(x, idx)
    gu = torch.nn.functional.linear(xs, mlp.gate_up.weight.cpu())
    gate, up = gu.chunk(2, -1)
    y = torch.nn.functional.linear(ofo.swiglu(gate, up), mlp.down.weight.cpu())
    want = torch.zeros_like(x).scatter_(1, idx.unsqueeze(-1).expand(-1, -1, D), y)
    from conftest import max_rel_err

    assert max_rel_err(out, want) < 1e-5
    assert max_rel_err(hr, h + want) < 1e-5
