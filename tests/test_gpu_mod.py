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


@pytest.mark.parametrize("bitonic", [False, True])
@pytest.mark.parametrize("B,L,k", [(1, 1, 1), (3, 64, 1), (3, 64, 64), (2, 1000, 999),
                                   (2, 16384, 12288), (5, 333, 100), (70, 128, 96),
                                   (3, 8192, 6144), (2, 8193, 7000), (4, 4096, 1)])
def test_topk_sizes(cuda, monkeypatch, B, L, k, bitonic):
    """Rows up to 8192 take the bucketed rank kernel, longer rows the
    device-wide radix sort; forced, the bitonic kernel takes rows up to
    16384."""
    if bitonic:
        monkeypatch.setenv("HYDRA_TOPK_BITONIC", "1")
    g = torch.Generator().manual_seed(L + k)
    _check_topk(omod.make_tied_logits(B, L, 0.05, g), k, cuda)


@pytest.mark.parametrize("pattern", ["all_equal", "two_values", "one_bin_wide", "ramp"])
def test_topk_degenerate_bins(cuda, pattern):
    """Score sets that fill one histogram bin (all equal, two values, many
    distinct values sharing their top bits) take the bucketed kernel's
    whole-row sort; a ramp spreads over many bins."""
    g = torch.Generator().manual_seed(11)
    L = 4096
    if pattern == "all_equal":
        s = torch.full((3, L), 0.25)
    elif pattern == "two_values":
        s = torch.where(torch.rand(3, L, generator=g) > 0.5, 1.0, -1.0)
    elif pattern == "one_bin_wide":
        s = 1.0 + torch.rand(3, L, generator=g) * 1e-3  # same top 14 key bits
    else:
        s = torch.linspace(-5, 5, L).repeat(3, 1)
    for k in (1, 1000, 3072, L):
        _check_topk(s, k, cuda)


@pytest.mark.parametrize("B,L,k", [(3, 16385, 12000), (2, 65536, 49152), (1, 100003, 1),
                                   (2, 40000, 40000), (4, 20000, 5000)])
def test_topk_long_rows(cuda, B, L, k):
    """Rows longer than 8192 take the radix sort in global memory."""
    g = torch.Generator().manual_seed(L + k)
    _check_topk(omod.make_tied_logits(B, L, 0.05, g), k, cuda)


def test_topk_long_rows_ties_specials_bf16(cuda):
    """Long rows: all-equal scores (ties resolved by index alone), NaN /
    +-inf / signed zeros sprinkled into random scores, and bf16 scores with
    a bf16 mask."""
    L = 30000
    g = torch.Generator().manual_seed(5)
    for k in (1, 7777, L):
        _check_topk(torch.full((2, L), -0.5), k, cuda)
    s = torch.randn(2, L, generator=g)
    pos = torch.randperm(L, generator=g)[:64]
    specials = torch.tensor([float("nan"), float("inf"), float("-inf"), 0.0, -0.0, 3.0, 3.0, -3.0])
    s[:, pos] = specials.repeat(8)
    for k in (1, 5, 12000):
        _check_topk(s, k, cuda)
    _check_topk(torch.randn(3, L, generator=g).to(torch.bfloat16), 20000, cuda, mask_dtype=torch.bfloat16)


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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scatter_add_repeated_indices(cuda, dtype):
    """scatter_add_by_indices keeps torch.scatter_add_'s semantics when
    indices repeat (ops.py:275-293): repeats accumulate in index order."""
    from hydra_amd.routing import scatter_add_by_indices

    g = torch.Generator().manual_seed(11)
    out = torch.randn(2, 40, 24, generator=g).to(dtype)
    vals = torch.randn(2, 60, 24, generator=g).to(dtype)
    idx = torch.randint(0, 40, (2, 60), generator=g)
    assert len(torch.unique(idx[0])) < 60  # repeats present
    want = out.clone().scatter_add_(1, idx.unsqueeze(-1).expand(-1, -1, 24), vals)
    got = out.to(cuda)
    scatter_add_by_indices(got, vals.to(cuda), idx.to(cuda))
    if dtype == torch.float32:
        assert torch.equal(got.cpu(), want)
    else:
        from conftest import max_rel_err

        assert max_rel_err(got.cpu(), want) < 2e-2


def test_gather_scatter_backward(cuda):
    """Gradients through gather_by_indices, scatter_replace and
    weighted_residual_scatter (weights included) equal autograd through
    torch.gather / scatter / index-add on the CPU (fp64 reference)."""
    from hydra_amd.routing import gather_by_indices, scatter_replace, weighted_residual_scatter

    g = torch.Generator().manual_seed(12)
    B, L, D, k = 2, 50, 16, 30
    x0 = torch.randn(B, L, D, generator=g)
    idx = torch.stack([torch.randperm(L, generator=g)[:k] for _ in range(B)])
    w0 = torch.rand(B, k, generator=g)
    G = torch.randn(B, L, D, generator=g)
    G2 = torch.randn(B, L, D, generator=g)

    def run(x, w, gather, scat_rep, scat_add, ix):
        xs = gather(x, ix) * 2.0 + 1.0
        out = x * 3.0
        out = scat_rep(out, xs, ix)
        h = x * 0.5
        h = scat_add(h, torch.tanh(xs), ix, w)
        return (out * G.to(out)).sum() + (h * G2.to(h)).sum()

    xd = x0.to(cuda).requires_grad_()
    wd = w0.to(cuda).requires_grad_()
    run(xd, wd, gather_by_indices, scatter_replace, weighted_residual_scatter, idx.to(cuda)).backward()

    def t_gather(x, ix):
        return torch.gather(x, 1, ix.unsqueeze(-1).expand(-1, -1, x.shape[-1]))

    def t_rep(out, v, ix):
        return out.scatter(1, ix.unsqueeze(-1).expand(-1, -1, out.shape[-1]), v)

    def t_add(h, v, ix, w):
        return h.scatter_add(1, ix.unsqueeze(-1).expand(-1, -1, h.shape[-1]), v * w[..., None])

    xr = x0.double().requires_grad_()
    wr = w0.double().requires_grad_()
    run(xr, wr, t_gather, t_rep, t_add, idx).backward()
    from conftest import max_rel_err

    assert max_rel_err(xd.grad.cpu(), xr.grad) < 1e-5
    assert max_rel_err(wd.grad.cpu(), wr.grad) < 1e-5


def test_mixture_of_depths_block_backward(cuda):
    """MixtureOfDepthsBlock (mixture_of_depths.py:283-297) trains: x and the
    wrapped block's weights get the gradients autograd gives the reference's
    gather / clone / scatter_ on the same selection."""
    from hydra_amd.routing import MixtureOfDepthsBlock

    g = torch.Generator().manual_seed(13)
    D = 32
    blk = torch.nn.Linear(D, D)
    mod = MixtureOfDepthsBlock(blk, D, capacity_ratio=0.5)
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.1)
    x0 = torch.randn(2, 64, D, generator=g)
    G = torch.randn(2, 64, D, generator=g)
    mod = mod.to(cuda)
    xd = x0.to(cuda).requires_grad_()
    (mod(xd) * G.to(cuda)).sum().backward()
    with torch.no_grad():
        _, idx, _ = mod.router(x0.to(cuda))
    idx = idx.cpu()
    ref_blk = torch.nn.Linear(D, D).double()
    ref_blk.load_state_dict({k: v.double().cpu() for k, v in blk.state_dict().items()})
    xr = x0.double().requires_grad_()
    ie = idx.unsqueeze(-1).expand(-1, -1, D)
    out = xr.clone().scatter(1, ie, ref_blk(torch.gather(xr, 1, ie)))
    (out * G.double()).sum().backward()
    from conftest import max_rel_err

    assert max_rel_err(xd.grad.cpu(), xr.grad) < 1e-5
    assert max_rel_err(blk.weight.grad.cpu(), ref_blk.weight.grad) < 1e-5
    assert max_rel_err(blk.bias.grad.cpu(), ref_blk.bias.grad) < 1e-5


def test_mod_mlp_ste_training_backward(cuda):
    """MoDMLPWrapper in training (the STE path, blocks.py:271-300): the MLP
    weights and x get the hard path's gradients, and the router gets exactly
    the aux loss's gradient (the straight-through term is multiplied by 0)."""
    from hydra_amd.layers import SwiGLUMLPFused
    from hydra_amd.routing import MoDMLPWrapper

    g = torch.Generator().manual_seed(14)
    D, Hd, L = 32, 48, 64
    mlp = SwiGLUMLPFused(D, Hd)
    wrap = MoDMLPWrapper(mlp, D, capacity_ratio=0.75, warmup_steps=0, aux_loss_weight=0.1)
    with torch.no_grad():
        for p in wrap.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.1)
    wrap.set_global_step(1)
    wrap = wrap.to(cuda).train()
    x0 = torch.randn(2, L, D, generator=g)
    G = torch.randn(2, L, D, generator=g)
    xd = x0.to(cuda).requires_grad_()
    out = wrap(xd)
    ((out * G.to(cuda)).sum() + wrap.get_aux_loss()).backward()
    idx = wrap._last_indices.cpu()

    ref = {k: v.double().cpu().requires_grad_() for k, v in wrap.state_dict().items()
           if v.is_floating_point() and not k.endswith("_aux_loss")}
    xr = x0.double().requires_grad_()
    ie = idx.unsqueeze(-1).expand(-1, -1, D)
    xs = torch.gather(xr, 1, ie)
    gate, up = torch.nn.functional.linear(xs, ref["mlp.gate_up.weight"]).chunk(2, -1)
    y = torch.nn.functional.linear(torch.nn.functional.silu(gate) * up, ref["mlp.down.weight"])
    o = torch.zeros_like(xr).scatter(1, ie, y)
    scores = torch.nn.functional.linear(xr, ref["mod_router.router.weight"],
                                        ref["mod_router.router.bias"]).squeeze(-1)
    probs = torch.sigmoid(scores.clamp(-10, 10))
    aux = 0.1 * ((probs.mean() - 0.75) ** 2 + 0.5 * torch.exp(-probs.var() / max(0.75 * 0.25 * 0.5, 0.01) * 5.0))
    ((o * G.double()).sum() + aux).backward()
    from conftest import max_rel_err

    assert max_rel_err(xd.grad.cpu(), xr.grad) < 1e-5
    for name, p in wrap.named_parameters():
        assert max_rel_err(p.grad.cpu(), ref[name].grad) < 1e-5, name
