"""GPU parity of the block compositions: the row kernels (embedding, residual
+ RMSNorm / AdaRMSNorm, MoR routing and update) against the oracle, the
config-1 block (embedding + HydraBlock with SwiGLU hidden 1365) at full size
against the oracle composition and the reference-run golden, and HydraModel
(MoR blocks with MoD, tied LM head) loaded from the checkpoint the
reference's save_checkpoint wrote, against its stored logits.
fp32 bar 1e-5, bf16 bar 2e-2 (normwise), indices and depths bit-exact."""
from __future__ import annotations

import ast
import math

import numpy as np
import pytest
import torch

from conftest import GOLDEN, bf16_from_bits, max_rel_err
from oracle import blocks as ob
from oracle import ccgqa as occ
from oracle import fused_ops as ofo

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim", [512, 1792, 100])
def test_embedding_lookup(cuda, dtype, dim):
    """Rows gathered bit for bit, ids clamped, times sqrt(dim) with one
    rounding; dim 100 takes the scalar path in bf16."""
    from hydra_amd.model.framework import embedding_lookup

    g = torch.Generator().manual_seed(dim)
    V = 1000
    table = (torch.randn(V, dim, generator=g) * 0.02).to(dtype)
    ids = torch.randint(0, V, (3, 77), generator=g)
    ids[0, 0], ids[1, 5], ids[2, 76] = -1, V, 10 * V
    got = embedding_lookup(table.to(cuda), ids.to(cuda), math.sqrt(dim)).cpu()
    want = ob.embedding(table, ids, math.sqrt(dim))
    assert torch.equal(got, want)


NORM_CASES = [(16384, 768), (1024, 512), (300, 1792), (64, 100)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,dim", NORM_CASES)
def test_residual_rms_norm(cuda, dtype, rows, dim):
    """h = x + r (rounded), y = RMSNorm(h) (fp32 inside) -- the fused pre-norm
    of HydraBlock -- and h = x + round(0.5 r) with no norm (HydraMoRBlock's
    scaled attention residual)."""
    from hydra_amd import _lib
    from hydra_amd.layers import residual_norm

    g = torch.Generator().manual_seed(rows + dim)
    x, r = (torch.randn(rows, dim, generator=g).to(dtype) for _ in range(2))
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(dtype)
    h, y = residual_norm(x.to(cuda), r=r.to(cuda), weight=w.to(cuda), norm=_lib.NORM_RMS, want_h=True)
    h_ref = x + r
    assert torch.equal(h.cpu(), h_ref)
    assert max_rel_err(y.cpu(), ofo.rms_norm(h_ref.float(), w.float())) < TOL[dtype]
    h2, _ = residual_norm(x.to(cuda), r=r.to(cuda), alpha=0.5, norm=_lib.NORM_NONE)
    assert torch.equal(h2.cpu(), x + 0.5 * r)
    # fp32 weight with 16-bit x: read in fp32 (the reference kernel's load)
    y32 = residual_norm(x.to(cuda), weight=w.float().to(cuda), norm=_lib.NORM_RMS)[1]
    assert max_rel_err(y32.cpu(), ofo.rms_norm(x.float(), w.float())) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,dim", NORM_CASES)
def test_ada_rms_norm_with_recursion_vectors(cuda, dtype, rows, dim):
    """AdaRMSNorm(current + recursion_bias + recursion_embed) in the input
    dtype (the MoR executor's pre-norm) against the oracle's torch ops."""
    from hydra_amd import _lib
    from hydra_amd.layers import AdaRMSNorm, residual_norm

    g = torch.Generator().manual_seed(rows * 3 + dim)
    x = torch.randn(rows, dim, generator=g).to(dtype)
    b1, b2 = ((0.02 * torch.randn(dim, generator=g)).to(dtype) for _ in range(2))
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(dtype)
    _, y = residual_norm(x.to(cuda), b1=b1.to(cuda), b2=b2.to(cuda), weight=w.to(cuda), norm=_lib.NORM_ADA)
    want = ob.ada_rms_norm(x + b1 + b2, w)
    err = max_rel_err(y.cpu(), want)
    assert err < TOL[dtype]
    if dtype == torch.bfloat16:
        # the rounding sequence is the reference's: almost every element is
        # bit-exact (a sum-order difference can move a row's mean by one ulp)
        assert (y.cpu() == want).float().mean() > 0.99
    m = AdaRMSNorm(dim).to(cuda, dtype)
    with torch.no_grad():
        m.weight.copy_(w)
        assert max_rel_err(m(x.to(cuda)).cpu(), ob.ada_rms_norm(x, w)) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("R,min_d", [(4, 0), (3, 0), (6, 2)])
def test_mor_route(cuda, dtype, R, min_d):
    from hydra_amd.routing.mixture_of_recursions import mor_route

    g = torch.Generator().manual_seed(R * 10 + min_d)
    logits = (3 * torch.randn(4, 999, generator=g)).to(dtype)
    d, p, l = mor_route(logits.to(cuda), R, min_d)
    dr, pr, lr = ob.mor_route(logits, R, min_d)
    assert max_rel_err(p.cpu(), pr) < TOL[dtype] and max_rel_err(l.cpu(), lr) < TOL[dtype]
    agree = (d.cpu() == dr).float().mean().item()
    if dtype == torch.float32:
        assert agree == 1.0
    else:  # a one-ulp tanh/sigmoid difference may cross a rounding boundary
        assert agree > 0.995


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mor_executor_update(cuda, dtype):
    from hydra_amd.routing.mixture_of_recursions import mor_update

    g = torch.Generator().manual_seed(9)
    B, L, D, R = 2, 333, 256, 4
    cur = torch.randn(B, L, D, generator=g).to(dtype)
    out = torch.randn(B, L, D, generator=g).to(dtype)
    depths = torch.randint(0, R, (B, L), generator=g)
    c_d, o_d = cur.to(cuda), out.to(cuda)
    c_ref, o_ref = cur.clone(), out.clone()
    for i in range(R):
        delta = torch.randn(B, L, D, generator=g).to(dtype)
        mor_update(c_d, delta.to(cuda), o_d, depths.to(cuda), i)
        c_ref = c_ref + delta * (depths >= i).unsqueeze(-1).to(dtype)
        o_ref = o_ref + c_ref * (depths == i).unsqueeze(-1).to(dtype)
    assert torch.equal(c_d.cpu(), c_ref) and torch.equal(o_d.cpu(), o_ref)


def _c1_modules(cfg, hidden, device, dtype, params):
    from hydra_amd.layers import SwiGLUMLPFused
    from hydra_amd.model.framework import HydraBlock

    blk = HydraBlock(dim=cfg.dim, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                     compression_factor=cfg.compression_factor, max_seq_len=cfg.max_seq_len)
    blk.mlp = SwiGLUMLPFused(cfg.dim, hidden)
    blk.load_state_dict({k: v for k, v in params.items() if k != "tok_emb.weight"})
    return blk.to(device=device, dtype=dtype).eval()


def _c1_forward(blk, table, ids, dim):
    from hydra_amd.model.framework import embedding_lookup

    with torch.no_grad():
        return blk(embedding_lookup(table, ids, math.sqrt(dim)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_c1_block_reference_golden(cuda, dtype):
    z = np.load(GOLDEN / "hydra_block_c1.npz")
    meta = ast.literal_eval(str(z["meta"]))
    p = {k[2:]: bf16_from_bits(z[k]) for k in z.files if k.startswith("w.")}
    cfg = occ.CCGQAConfig(dim=meta["dim"], n_heads=meta["n_heads"], n_kv_heads=meta["n_kv_heads"],
                          compression_factor=meta["compression_factor"], max_seq_len=64)
    blk = _c1_modules(cfg, meta["hidden"], cuda, dtype, p)
    got = _c1_forward(blk, p["tok_emb.weight"].to(cuda, dtype), torch.from_numpy(z["ids"]).to(cuda), cfg.dim)
    assert max_rel_err(got.float().cpu(), torch.from_numpy(z["out"])) < TOL[dtype]


def test_c1_full_shape_fp32(cuda):
    """Config 1 at its own shape: ids [2, 512] over vocab 32000, dim 512,
    8/2 heads of 16, SwiGLU hidden 1365, N(0, 0.02) weights, fp32."""
    g = torch.Generator().manual_seed(0)
    cfg = occ.CCGQAConfig(dim=512, n_heads=8, n_kv_heads=2, compression_factor=4, max_seq_len=512)
    ids = torch.randint(0, 32000, (2, 512), generator=g)
    p = occ.init_params(cfg, g, temperature=4.0)
    p = {"attention." + k: v for k, v in p.items()}
    p["norm1.weight"] = torch.ones(512)
    p["norm2.weight"] = torch.ones(512)
    p["mlp.gate_up.weight"] = torch.randn(2 * 1365, 512, generator=g) * 0.02
    p["mlp.down.weight"] = torch.randn(512, 1365, generator=g) * 0.02
    p["tok_emb.weight"] = torch.randn(32000, 512, generator=g) * 0.02
    blk = _c1_modules(cfg, 1365, cuda, torch.float32, p)
    got = _c1_forward(blk, p["tok_emb.weight"].to(cuda), ids.to(cuda), 512).cpu()
    want = ob.c1_forward(p, ids, cfg)
    assert max_rel_err(got, want) < 1e-5


def _model_from_checkpoint(device, dtype):
    from hydra_amd.model.framework import HydraModel
    from hydra_amd.training import load_module_from_checkpoint

    z = np.load(GOLDEN / "hydra_model_fwd.npz")
    meta = ast.literal_eval(str(z["meta"]))
    m = HydraModel(vocab_size=meta["vocab_size"], dim=meta["dim"], n_mor_blocks=meta["n_mor_blocks"],
                   recursions_per_block=meta["recursions_per_block"], n_heads=meta["n_heads"],
                   n_kv_heads=meta["n_kv_heads"], compression_factor=meta["compression_factor"],
                   mlp_ratio=meta["mlp_ratio"], max_seq_len=meta["max_seq_len"],
                   mod_capacity=meta["mod_capacity"], adaptive=True, tie_weights=True)
    missing, unexpected = load_module_from_checkpoint(m, GOLDEN / "hydra_model_ckpt.pt")
    assert not missing and not unexpected
    m.set_global_step(meta["global_step"])
    return m.to(device=device, dtype=dtype).eval(), z, meta


def test_hydra_model_reference_checkpoint_fp32(cuda):
    """Checkpoint written by the reference's save_checkpoint, loaded through
    load_module_from_checkpoint, forward on the GPU against the logits the
    reference model produced (MoD in the middle block, MoR depths 0..2)."""
    m, z, _ = _model_from_checkpoint(cuda, torch.float32)
    ids = torch.from_numpy(z["ids"]).to(cuda)
    with torch.no_grad():
        logits = m(ids).cpu()
        hidden = m.forward_hidden(ids).cpu()
    assert max_rel_err(logits, torch.from_numpy(z["logits"])) < 1e-5
    assert max_rel_err(hidden, torch.from_numpy(z["hidden"])) < 1e-5


def test_hydra_model_bf16_decisions(cuda):
    """bf16: the device's routing decisions (MoR depths, MoD selections) are
    captured and given to the oracle, which runs the same model in bf16 on
    the CPU; logits within 2e-2, and the decisions agree with the oracle's
    own on all but near-tied tokens."""
    from hydra_amd.training import read_checkpoint

    m, z, meta = _model_from_checkpoint(cuda, torch.bfloat16)
    ids = torch.from_numpy(z["ids"])
    rec = [dict() for _ in m.layers]
    calls = [0] * len(m.layers)

    def hook(li):
        def fn(mod, inp, out):
            rec[li][f"mod_idx{calls[li]}"] = mod._last_indices.cpu()
            calls[li] += 1
        return fn

    hs = [l.mod_mlp_wrapper.register_forward_hook(hook(i)) for i, l in enumerate(m.layers)
          if l.mod_mlp_wrapper is not None]
    with torch.no_grad():
        logits = m(ids.to(cuda)).float().cpu()
    for h in hs:
        h.remove()
    for i, l in enumerate(m.layers):
        rec[i]["depths"] = l._last_depths.cpu()
    params = {k: v.to(torch.bfloat16) if v.is_floating_point() else v
              for k, v in read_checkpoint(GOLDEN / "hydra_model_ckpt.pt")["model"].items()}
    cfg = ob.ModelConfig(vocab_size=meta["vocab_size"], dim=meta["dim"], n_mor_blocks=meta["n_mor_blocks"],
                         recursions_per_block=meta["recursions_per_block"], n_heads=meta["n_heads"],
                         n_kv_heads=meta["n_kv_heads"], compression_factor=meta["compression_factor"],
                         max_seq_len=meta["max_seq_len"], mod_capacity=meta["mod_capacity"])
    traces = []
    want = ob.hydra_model(params, ids, cfg, traces=traces, forces=rec).float()
    assert max_rel_err(logits, want) < 2e-2
    # the oracle's own decisions (not forced) agree with the device's on all
    # but near-tied tokens: depths per token, MoD selections as sets
    free = []
    ob.hydra_model(params, ids, cfg, traces=free)
    for i in range(cfg.n_mor_blocks):
        assert (rec[i]["depths"] == free[i]["depths"]).float().mean() > 0.95
        for r in range(cfg.recursions_per_block):
            key = f"mod_idx{r}"
            if key not in rec[i]:
                continue
            k = rec[i][key].shape[1]
            from oracle import mod as omod
            own = torch.from_numpy(omod.topk_desc_lowest_index(free[i][f"mod_scores{r}"].float().numpy(), k))
            for b in range(own.shape[0]):
                inter = len(set(own[b].tolist()) & set(rec[i][key][b].tolist()))
                assert inter >= 0.95 * k


def _capture_decisions(m):
    """Forward hooks that record each layer's MoD selections (per call) and,
    after the forward, its MoR depths: the forcing input of
    oracle.blocks.hydra_model."""
    rec = [dict() for _ in m.layers]
    calls = [0] * len(m.layers)

    def hook(li):
        def fn(mod, inp, out):
            rec[li][f"mod_idx{calls[li]}"] = mod._last_indices.cpu()
            calls[li] += 1
        return fn

    hs = [l.mod_mlp_wrapper.register_forward_hook(hook(i)) for i, l in enumerate(m.layers)
          if l.mod_mlp_wrapper is not None]

    def finish():
        for h in hs:
            h.remove()
        for i, l in enumerate(m.layers):
            rec[i]["depths"] = l._last_depths.cpu()
        return rec
    return finish


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hydra_model_c5_layout(cuda, dtype):
    """Config 5's layer widths at reduced depth and length: dim 1792, 28 q /
    4 kv heads of 16 (groups of 7), latent 448, mlp_ratio 3.6 (hidden
    6656), 3 MoR blocks x 2 recursions with MoD (capacity 0.75) on the
    middle block, tied LM head (vocab 1000).  The device's routing
    decisions are handed to the oracle (oracle/blocks.py:hydra_model,
    restating model.py:408-502 and blocks.py:431-756), which runs the same
    weights on the CPU in the same dtype; logits within 1e-5 (fp32) /
    2e-2 (bf16)."""
    from hydra_amd.model.framework import HydraModel

    torch.manual_seed(5)
    kw = dict(vocab_size=1000, dim=1792, n_mor_blocks=3, recursions_per_block=2, n_heads=28,
              n_kv_heads=4, compression_factor=4, max_seq_len=128, mod_capacity=0.75)
    m = HydraModel(mlp_ratio=3.6, adaptive=True, tie_weights=True, **kw)
    m.set_global_step(10000)
    params = {k: v.detach().clone() for k, v in m.state_dict().items()}
    if dtype != torch.float32:
        params = {k: v.to(dtype) if v.is_floating_point() else v for k, v in params.items()}
    m = m.to(device=cuda, dtype=dtype).eval()
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, 1000, (2, 64), generator=g)
    finish = _capture_decisions(m)
    with torch.no_grad():
        logits = m(ids.to(cuda)).float().cpu()
    rec = finish()
    assert any(k.startswith("mod_idx") for k in rec[1]), "MoD ran on the middle block"
    cfg = ob.ModelConfig(**kw)
    want = ob.hydra_model(params, ids, cfg, forces=rec).float()
    assert max_rel_err(logits, want) < TOL[dtype]
