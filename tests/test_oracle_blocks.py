"""Pins of oracle/blocks.py and of the chunked-CE clamp rule -- CPU only.

The compositions (config-1 block, HydraModel with MoR + MoD) are pinned by
golden vectors written by running the reference (tests/golden/make_golden.py):
its HydraBlock forward after _safe_embedding_lookup, and a HydraModel saved
through its own save_checkpoint with its forward logits.  The pieces are
also checked against closed forms and invariants chosen so that a dropped
term or a wrong rounding point fails."""
from __future__ import annotations

import ast
import math

import numpy as np
import torch
import torch.nn.functional as F

from conftest import GOLDEN, bf16_from_bits, max_rel_err
from oracle import blocks as ob
from oracle import ccgqa as occ
from oracle import fused_ops as ofo


def _golden_params(z, prefix="w."):
    return {k[len(prefix):]: bf16_from_bits(z[k]) for k in z.files if k.startswith(prefix)}


def test_c1_block_matches_reference_golden():
    z = np.load(GOLDEN / "hydra_block_c1.npz")
    meta = ast.literal_eval(str(z["meta"]))
    p = _golden_params(z)
    cfg = occ.CCGQAConfig(dim=meta["dim"], n_heads=meta["n_heads"], n_kv_heads=meta["n_kv_heads"],
                          compression_factor=meta["compression_factor"], max_seq_len=64)
    ids = torch.from_numpy(z["ids"])
    h0 = ob.embedding(p["tok_emb.weight"], ids, math.sqrt(meta["dim"]))
    assert torch.equal(h0, torch.from_numpy(z["h0"]))  # clamp + scale, bit for bit
    out = ob.c1_forward(p, ids, cfg)
    assert max_rel_err(out, torch.from_numpy(z["out"])) < 1e-6


def _model_case():
    from hydra_amd.training import read_checkpoint

    ck = read_checkpoint(GOLDEN / "hydra_model_ckpt.pt")
    z = np.load(GOLDEN / "hydra_model_fwd.npz")
    meta = ast.literal_eval(str(z["meta"]))
    cfg = ob.ModelConfig(vocab_size=meta["vocab_size"], dim=meta["dim"], n_mor_blocks=meta["n_mor_blocks"],
                         recursions_per_block=meta["recursions_per_block"], n_heads=meta["n_heads"],
                         n_kv_heads=meta["n_kv_heads"], compression_factor=meta["compression_factor"],
                         max_seq_len=meta["max_seq_len"], mod_capacity=meta["mod_capacity"])
    return ck, z, cfg


def test_hydra_model_matches_reference_checkpoint_and_logits():
    ck, z, cfg = _model_case()
    assert ck["step"] == 7 and set(ck["rng_state"]) >= {"python", "torch", "numpy"}
    ids = torch.from_numpy(z["ids"])
    traces = []
    logits = ob.hydra_model(ck["model"], ids, cfg, traces=traces)
    assert max_rel_err(logits, torch.from_numpy(z["logits"])) < 1e-5
    hidden = ob.hydra_model(ck["model"], ids, cfg, return_hidden=True)
    assert max_rel_err(hidden, torch.from_numpy(z["hidden"])) < 1e-5
    # the case exercises every routing branch: several depths per block and
    # MoD (k < L) in the middle block
    for tr in traces:
        assert len(torch.unique(tr["depths"])) >= 2
    assert "mod_scores0" in traces[1] and "mod_scores0" not in traces[0]


def test_hydra_model_mod_and_mor_are_load_bearing():
    """Dropping MoD (dense MLP in the middle block) or the MoR depth mask
    (every token through every recursion) moves the logits: the golden
    checks both mechanisms, not just the dense path."""
    ck, z, cfg = _model_case()
    ids = torch.from_numpy(z["ids"])
    ref = torch.from_numpy(z["logits"])
    cfg.mod_enabled = False
    assert max_rel_err(ob.hydra_model(ck["model"], ids, cfg), ref) > 1e-3
    cfg.mod_enabled = True
    forces = [{"depths": torch.full(ids.shape, cfg.recursions_per_block - 1)} for _ in range(cfg.n_mor_blocks)]
    assert max_rel_err(ob.hydra_model(ck["model"], ids, cfg, forces=forces), ref) > 1e-3


def test_ada_rms_norm_rounding_points():
    """fp32: the closed form x / sqrt(mean(x^2) + eps) * w.  bf16: each step
    is rounded (the square, the mean, the sum with eps, the rsqrt, the two
    products), which differs from the fp32-inside RMSNorm on some elements."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(6, 40, generator=g, dtype=torch.float64)
    w = 1 + 0.1 * torch.randn(40, generator=g, dtype=torch.float64)
    want = x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * w
    assert torch.allclose(ob.ada_rms_norm(x, w), want, rtol=1e-12)
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16)
    got = ob.ada_rms_norm(xb, wb)
    assert got.dtype == torch.bfloat16
    sq = (xb.float() ** 2).to(torch.bfloat16).float()
    m = sq.mean(-1, keepdim=True).to(torch.bfloat16).float()
    s = torch.rsqrt((m + 1e-6).to(torch.bfloat16).float()).to(torch.bfloat16).float()
    step = ((xb.float() * s).to(torch.bfloat16).float() * wb.float()).to(torch.bfloat16)
    assert torch.equal(got, step)
    assert not torch.equal(got, ofo.rms_norm(xb.float(), wb.float()).to(torch.bfloat16))


def test_mor_route_known_answers():
    """logit 0 -> tanh 0 -> p = 1/2 -> depth round((R-1)/2) (half to even);
    large logits saturate at tanh = 1 -> p = sigmoid(3); depths monotone."""
    for R in (2, 3, 4, 5):
        d, p, l = ob.mor_route(torch.zeros(1, 1), R)
        assert p.item() == 0.5 and l.item() == 0.0
        assert d.item() == int(np.round((R - 1) / 2))
    d, p, _ = ob.mor_route(torch.tensor([[50.0, -50.0]]), 4)
    assert math.isclose(p[0, 0].item(), 1 / (1 + math.exp(-3)), rel_tol=1e-6)
    assert d.tolist() == [[round(3 / (1 + math.exp(-3)))], ] or d[0, 0].item() == 3
    xs = torch.linspace(-20, 20, 401)[None]
    d, _, _ = ob.mor_route(xs, 4)
    assert (d[0, 1:] >= d[0, :-1]).all()
    d, _, _ = ob.mor_route(xs, 4, min_d=1)
    assert d.min() >= 1


def test_mor_executor_state_machine():
    """Token with depth d: its state moves through recursions 0..d and the
    output holds the state after recursion d (brute force per token)."""
    g = torch.Generator().manual_seed(6)
    B, L, D, R = 2, 5, 3, 4
    x = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    depths = torch.randint(0, R, (B, L), generator=g)
    rb = torch.randn(R, 1, 1, D, generator=g, dtype=torch.float64)
    re = torch.randn(R, D, generator=g, dtype=torch.float64)
    mats = [torch.randn(D, D, generator=g, dtype=torch.float64) for _ in range(R)]
    out = ob.mor_executor(x, depths, None, lambda y, i: y @ mats[i], lambda t: torch.tanh(t), rb, re, R)
    for b in range(B):
        for t in range(L):
            c = x[b, t].clone()
            for i in range(depths[b, t].item() + 1):
                c = c + torch.tanh(c + rb[i, 0, 0] + re[i]) @ mats[i]
            assert torch.allclose(out[b, t], c, rtol=1e-12)


def test_chunked_ce_matches_reference_outputs():
    """The reference's ChunkedCrossEntropyFunction outputs (golden): with an
    out-of-range target it clamps the whole vector, so the ignore entries
    become class 0 and count; without one, ignore entries stay ignored."""
    z = np.load(GOLDEN / "chunked_ce_cpu.npz")
    h, w = bf16_from_bits(z["h"]), bf16_from_bits(z["w"])
    go = float(z["grad_output"])
    for name in ("mixed", "ignore_only"):
        t = torch.from_numpy(z[f"{name}_targets"])
        loss, gh, gw = ofo.chunked_cross_entropy(h, w, t, grad_output=go)
        assert abs(loss.item() - float(z[f"{name}_loss"])) < 1e-5 * abs(loss.item())
        assert max_rel_err(gh, torch.from_numpy(z[f"{name}_grad_h"])) < 1e-5
        assert max_rel_err(gw, torch.from_numpy(z[f"{name}_grad_w"])) < 1e-5
    # the mixed case really differs from clamping the valid targets only
    t = torch.from_numpy(z["mixed_targets"])
    valid = t != -100
    loss_valid_only = F.cross_entropy((h.double() @ w.double().t()).reshape(-1, w.shape[0]),
                                      torch.where(valid, t.clamp(0, 99), torch.full_like(t, -100)).reshape(-1),
                                      ignore_index=-100)
    assert abs(loss_valid_only.item() - float(z["mixed_loss"])) > 1e-4
