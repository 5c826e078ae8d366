"""Pins of the CPU oracle (oracle/) -- CPU only.

Each oracle function is checked against something independent of its own
formula: a brute-force fp64 loop, a closed form at a chosen point, an
invariant, a library routine it must agree with, the reference's own
equivalence tests (restated), or the golden vectors written by running the
reference (tests/golden/make_golden.py).  The checks are chosen so a dropped
term, a flipped sign, a wrong tap order or a transposed operand fails one.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN, bf16_from_bits, max_rel_err
from oracle import ccgqa as occ
from oracle import fused_ops as ofo
from oracle import mod as omod


# ---------------------------------------------------------------- fused ops
def test_rms_norm_bruteforce_and_invariant():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 7, 33, generator=g, dtype=torch.float64)
    w = 1 + 0.1 * torch.randn(33, generator=g, dtype=torch.float64)
    y = ofo.rms_norm(x, w, 1e-6)
    for r in range(3):
        for s in range(7):
            ms = sum(float(v) ** 2 for v in x[r, s]) / 33
            ref = [float(x[r, s, i]) / math.sqrt(ms + 1e-6) * float(w[i]) for i in range(33)]
            assert np.allclose(y[r, s].numpy(), ref, rtol=1e-12, atol=1e-12)
    # invariant: rms(y / w) == 1 (eps negligible here)
    rms = (y / w).pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-6)
    # the Triton-arithmetic variant agrees in fp32
    assert max_rel_err(ofo.rms_norm_fp32(x.float(), w.float()), y) < 1e-6


def test_rope_known_answer_and_norm():
    # One pair rotated by a known angle: position s, pair i has angle s * theta^(-2i/D).
    D, S = 4, 3
    cos, sin = ofo.rope_cache(D, S)
    x = torch.zeros(1, 1, S, D)
    x[..., 0] = 1.0  # pair 0 = (1, 0)
    x[..., 3] = 1.0  # pair 1 = (0, 1)
    y = ofo.rope(x, cos, sin)
    for s in range(S):
        a0 = s * 1.0
        a1 = s * 10000.0 ** (-2 / D)
        # (1,0) -> (cos a, sin a); (0,1) -> (-sin a, cos a)
        assert math.isclose(y[0, 0, s, 0].item(), math.cos(a0), abs_tol=1e-6)
        assert math.isclose(y[0, 0, s, 1].item(), math.sin(a0), abs_tol=1e-6)
        assert math.isclose(y[0, 0, s, 2].item(), -math.sin(a1), abs_tol=1e-6)
        assert math.isclose(y[0, 0, s, 3].item(), math.cos(a1), abs_tol=1e-6)
    # position 0 is the identity; every pair keeps its norm
    g = torch.Generator().manual_seed(1)
    xr = torch.randn(2, 3, 9, 16, generator=g)
    cos, sin = ofo.rope_cache(16, 9)
    yr = ofo.rope(xr, cos, sin)
    assert torch.equal(yr[:, :, 0], xr[:, :, 0])
    pn = lambda t: t.reshape(*t.shape[:-1], -1, 2).norm(dim=-1)
    assert torch.allclose(pn(yr), pn(xr), atol=1e-5)


def test_rope_matches_reference_fallback_test():
    """tests/test_ccgqa_attention_refactors.py:161-196 restated: the even/odd
    slot formula, bit-exact."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 4, 32, 16, generator=g)
    cos, sin = ofo.rope_cache(16, 128)
    c, s = cos[:, :, :32], sin[:, :, :32]
    ref = torch.empty_like(x)
    x1, x2 = x[..., ::2], x[..., 1::2]
    ref[..., ::2] = x1 * c - x2 * s
    ref[..., 1::2] = x1 * s + x2 * c
    assert torch.equal(ofo.rope(x, cos, sin), ref)


def test_swiglu_closed_form():
    g = torch.Generator().manual_seed(2)
    gate = torch.randn(5, 17, generator=g, dtype=torch.float64) * 4
    up = torch.randn(5, 17, generator=g, dtype=torch.float64)
    ref = gate / (1 + torch.exp(-gate)) * up
    assert torch.allclose(ofo.swiglu(gate, up), ref, rtol=1e-12, atol=1e-12)
    assert ofo.swiglu(torch.tensor([0.0]), torch.tensor([5.0])).item() == 0.0
    assert max_rel_err(ofo.swiglu_fp32(gate.float(), up.float()), ref) < 1e-6


def test_qk_norm_norms():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 4, 5, 16, generator=g, dtype=torch.float64)
    k = torch.randn(2, 2, 5, 16, generator=g, dtype=torch.float64)
    qn, kn = ofo.qk_norm(q, k, 3.0, 0.5)
    assert torch.allclose(qn.norm(dim=-1), torch.full((2, 4, 5), 3.0, dtype=torch.float64))
    assert torch.allclose(kn.norm(dim=-1), torch.full((2, 2, 5), 1.5, dtype=torch.float64))
    # direction preserved
    assert torch.allclose(qn / 3.0 * q.norm(dim=-1, keepdim=True), q)
    qt, kt = ofo.qk_norm_triton_formula(q.float(), k.float(), 3.0, 0.5)
    assert max_rel_err(qt, qn) < 1e-6 and max_rel_err(kt, kn) < 1e-6


def test_fused_ops_golden():
    d = np.load(GOLDEN / "fused_ops_cpu.npz")
    x, w = bf16_from_bits(d["x"]), bf16_from_bits(d["w"])
    assert torch.equal(ofo.rms_norm(x, w, float(d["eps"])), torch.from_numpy(d["rms_out"]))
    gate, up = bf16_from_bits(d["gate"]), bf16_from_bits(d["up"])
    assert torch.equal(ofo.swiglu(gate, up), torch.from_numpy(d["swiglu_out"]))
    xr = bf16_from_bits(d["xr"])
    cos, sin = torch.from_numpy(d["cos"]), torch.from_numpy(d["sin"])
    assert torch.equal(ofo.rope(xr, cos, sin), torch.from_numpy(d["rope_out"]))
    q, k = bf16_from_bits(d["q"]), bf16_from_bits(d["k"])
    qn, kn = ofo.qk_norm(q, k, float(d["scale"]), float(d["temperature"]))
    assert torch.equal(qn, torch.from_numpy(d["qn_out"]))
    assert torch.equal(kn, torch.from_numpy(d["kn_out"]))


# -------------------------------------------------------------------- CCGQA
def _conv_bruteforce(x, w1, w2, groups1):
    """fp64 triple loop: y[s,o] = sum_t sum_c w[o,c,t] * u[s+t-2, c], u = 0 for s<0."""
    B, N, C = x.shape
    cpg = C // groups1
    y1 = torch.zeros(B, N, C, dtype=torch.float64)
    for b in range(B):
        for s in range(N):
            for o in range(C):
                g = o // cpg
                acc = 0.0
                for t in range(3):
                    src = s + t - 2
                    if src < 0:
                        continue
                    for c in range(cpg):
                        acc += float(w1[o, c, t]) * float(x[b, src, g * cpg + c])
                y1[b, s, o] = acc
    y2 = torch.zeros(B, N, C, dtype=torch.float64)
    for b in range(B):
        for s in range(N):
            for o in range(C):
                acc = 0.0
                for t in range(3):
                    src = s + t - 2
                    if src < 0:
                        continue
                    for c in range(C):
                        acc += float(w2[o, c, t]) * float(y1[b, src, c])
                y2[b, s, o] = acc
    return y2


def test_causal_conv_seq_bruteforce_and_causality():
    g = torch.Generator().manual_seed(4)
    B, N, C, G = 2, 7, 6, 3
    x = torch.randn(B, N, C, generator=g, dtype=torch.float64)
    w1 = torch.randn(C, C // G, 3, generator=g, dtype=torch.float64)
    w2 = torch.randn(C, C, 3, generator=g, dtype=torch.float64)
    y = occ.causal_conv_seq(x, w1, w2, G)
    assert torch.allclose(y, _conv_bruteforce(x, w1, w2, G), rtol=1e-10, atol=1e-10)
    # causality: perturbing token 4 leaves outputs 0..3 unchanged, changes 4..6
    x2 = x.clone()
    x2[:, 4] += 1.0
    y2 = occ.causal_conv_seq(x2, w1, w2, G)
    assert torch.equal(y2[:, :4], y[:, :4])
    assert not torch.allclose(y2[:, 4:], y[:, 4:])


def _cfg(**kw):
    base = dict(dim=64, n_heads=4, n_kv_heads=2, compression_factor=2, max_seq_len=128)
    base.update(kw)
    return occ.CCGQAConfig(**base)


def test_value_shift_matches_padcat():
    """tests/test_ccgqa_attention_refactors.py:109-132 restated."""
    cfg = _cfg(use_rope=False, use_qk_norm=False, use_convs=False, use_qk_mean=False)
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(2, 32, cfg.latent_dim + 2 * cfg.kv_dim, generator=g)
    _, _, v = occ.prep({}, qkv, cfg)
    L, K = cfg.latent_dim, cfg.kv_dim
    v_curr, v_prev = qkv[..., L + K:L + K + K // 2], qkv[..., L + K + K // 2:]
    v_ref = torch.cat([v_curr, F.pad(v_prev[:, :-1, :], (0, 0, 1, 0))], dim=-1)
    v_ref = v_ref.view(2, 32, cfg.n_kv_heads, cfg.head_dim).transpose(1, 2)
    assert torch.equal(v, v_ref)


def test_qk_mean_headspace_matches_expand():
    """tests/test_ccgqa_attention_refactors.py:135-158 restated."""
    cfg = _cfg(use_rope=False, use_qk_norm=False, use_convs=False, use_value_shift=False)
    g = torch.Generator().manual_seed(0)
    B, S = 2, 32
    L, K, hd = cfg.latent_dim, cfg.kv_dim, cfg.head_dim
    qkv = torch.randn(B, S, L + 2 * K, generator=g)
    q, k, _ = occ.prep({}, qkv, cfg)
    q0, k0 = qkv[..., :L], qkv[..., L:L + K]
    qm = q0.view(B, S, cfg.n_heads, hd).mean(2)
    km = k0.view(B, S, cfg.n_kv_heads, hd).mean(2)
    q_old = q0 + 0.5 * km.unsqueeze(2).expand(-1, -1, cfg.n_heads, -1).reshape(B, S, L)
    k_old = k0 + 0.5 * qm.unsqueeze(2).expand(-1, -1, cfg.n_kv_heads, -1).reshape(B, S, K)
    assert torch.equal(q, q_old.view(B, S, cfg.n_heads, hd).transpose(1, 2))
    assert torch.equal(k, k_old.view(B, S, cfg.n_kv_heads, hd).transpose(1, 2))


def test_qk_mean_uses_preconv_values():
    """The coupling term comes from q/k before the convs: with zero conv
    weights the conv path contributes nothing and q == 0.5 * mean(k_pre)."""
    cfg = _cfg(use_rope=False, use_qk_norm=False, use_value_shift=False)
    g = torch.Generator().manual_seed(5)
    params = occ.init_params(cfg, g)
    for n in list(params):
        if "conv" in n:
            params[n] = torch.zeros_like(params[n])
    qkv = torch.randn(1, 6, cfg.latent_dim + 2 * cfg.kv_dim, generator=g)
    q, _, _ = occ.prep(params, qkv, cfg)
    L, K, hd = cfg.latent_dim, cfg.kv_dim, cfg.head_dim
    km = qkv[..., L:L + K].view(1, 6, cfg.n_kv_heads, hd).mean(2)
    assert torch.allclose(q, (0.5 * km).unsqueeze(1).expand(-1, cfg.n_heads, -1, -1))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("use_mask", [False, True])
def test_attention_bruteforce(causal, use_mask):
    g = torch.Generator().manual_seed(6)
    B, Hq, Hkv, S, hd = 2, 4, 2, 9, 8
    q = torch.randn(B, Hq, S, hd, generator=g)
    k = torch.randn(B, Hkv, S, hd, generator=g)
    v = torch.randn(B, Hkv, S, hd, generator=g)
    mask = None
    if use_mask:
        mask = (torch.rand(B, S, generator=g) > 0.3).long()
        mask[:, 0] = 1
    if use_mask and causal:
        # the reference hands "True = masked" to SDPA (True = attend): visible
        # keys are t > s or padded ones.
        out = occ.attention(q, k, v, causal=True, mask=mask)
        Bm = mask.clone()
        ref = torch.zeros(B, Hq, S, hd, dtype=torch.float64)
        for b in range(B):
            for h in range(Hq):
                for s in range(S):
                    ts = [t for t in range(S) if t > s or Bm[b, t] == 0]
                    if not ts:
                        continue
                    lg = torch.stack([(q[b, h, s].double() * k[b, h // 2, t].double()).sum() / math.sqrt(hd) for t in ts])
                    p = torch.softmax(lg, 0)
                    ref[b, h, s] = sum(p[i] * v[b, h // 2, t].double() for i, t in enumerate(ts))
        assert max_rel_err(out, ref) < 1e-5
        return
    if use_mask:
        pytest.skip("padding mask is only defined together with causality in the reference")
    out = occ.attention(q, k, v, causal=causal)
    ref = occ.attention_bruteforce(q, k, v, causal=causal)
    assert max_rel_err(out, ref) < 1e-5


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("use_mask", [False, True])
def test_attention_key_padding_vectorised(causal, use_mask):
    """The vectorised key-padding softmax equals the triple loop, including
    rows that see no key (zeros)."""
    g = torch.Generator().manual_seed(8)
    B, Hq, Hkv, S, hd = 2, 6, 2, 11, 8
    q = torch.randn(B, Hq, S, hd, generator=g)
    k = torch.randn(B, Hkv, S, hd, generator=g)
    v = torch.randn(B, Hkv, S, hd, generator=g)
    mask = None
    if use_mask:
        mask = (torch.rand(B, S, generator=g) > 0.4).long()
        mask[0, :4] = 0  # causal rows 0..3 of batch 0 see no key
        mask[1, 0] = 1
    out = occ.attention_key_padding(q, k, v, causal=causal, mask=mask)
    ref = occ.attention_bruteforce(q, k, v, causal=causal, mask=mask)
    assert torch.allclose(out, ref, rtol=1e-12, atol=1e-12)
    if use_mask and causal:
        assert torch.count_nonzero(out[0, :, :4]) == 0


def test_attention_gqa_equals_repeat_interleave():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 6, 10, 8, generator=g)
    k = torch.randn(1, 2, 10, 8, generator=g)
    v = torch.randn(1, 2, 10, 8, generator=g)
    out = occ.attention(q, k, v, causal=True)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(3, 1), v.repeat_interleave(3, 1), is_causal=True)
    assert torch.equal(out, ref)


GOLDEN_CCGQA = sorted(GOLDEN.glob("ccgqa_*.npz"))


def load_ccgqa_golden(path):
    d = np.load(path)
    meta = dict(eval(str(d["meta"])))  # written by make_golden.py as a repr of sorted items
    B, S, msl = meta.pop("B"), meta.pop("S"), meta.pop("max_seq_len")
    cfg = occ.CCGQAConfig(max_seq_len=msl, **meta)
    params = {k[2:]: bf16_from_bits(d[k]) for k in d.files if k.startswith("w.")}
    x = bf16_from_bits(d["x"])
    mask = torch.from_numpy(d["mask"]).long() if "mask" in d.files else None
    return cfg, params, x, mask, torch.from_numpy(d["out"])


@pytest.mark.parametrize("path", GOLDEN_CCGQA, ids=[p.stem for p in GOLDEN_CCGQA])
def test_ccgqa_forward_golden(path):
    cfg, params, x, mask, out = load_ccgqa_golden(path)
    got = occ.forward(params, x, cfg, mask=mask)
    assert max_rel_err(got, out) < 1e-6


def test_flop_figures_match_baseline():
    """The algorithmic work the roofline is computed from (config 3)."""
    cfg = occ.CCGQAConfig(dim=1024, n_heads=4, n_kv_heads=1, compression_factor=4)
    f = occ.flops(cfg, 4, 4096)
    assert f["core"] == 34_368_126_976
    assert abs(f["total"] / 1e9 - 64.70) < 0.01


# ---------------------------------------------------------------------- MoD
def test_topk_bruteforce_ties_nan_signed_zero():
    rows = np.array([
        [1.0, 3.0, 3.0, -1.0, 3.0, 0.5],
        [0.0, -0.0, 0.0, -0.0, 1.0, -1.0],
        [np.nan, 2.0, np.nan, -np.inf, np.inf, 2.0],
        [np.inf, 2.0, np.nan, -np.inf, np.inf, np.nan],
    ])
    for k in range(1, 7):
        assert np.array_equal(omod.topk_desc_lowest_index(rows, k), omod.topk_desc_bruteforce(rows, k))
    assert omod.topk_desc_lowest_index(rows, 3)[0].tolist() == [1, 2, 4]
    assert omod.topk_desc_lowest_index(rows, 4)[1].tolist() == [4, 0, 1, 2]
    assert omod.topk_desc_lowest_index(rows, 4)[2].tolist() == [0, 2, 4, 1]
    # NaN ranks above +inf whatever the positions (torch.topk's order)
    assert omod.topk_desc_lowest_index(rows, 4)[3].tolist() == [2, 5, 0, 4]
    t = torch.topk(torch.from_numpy(rows[3]), 4).values
    assert np.isnan(t[0].item()) and np.isnan(t[1].item()) and t[2].item() == np.inf


def test_topk_value_sequence_matches_torch():
    g = torch.Generator().manual_seed(8)
    s = omod.make_tied_logits(4, 512, 0.05, g)
    for k in (1, 100, 384, 512):
        ours = omod.topk_desc_lowest_index(s.numpy(), k)
        vals = torch.topk(s, k, dim=-1).values
        assert torch.equal(torch.gather(s, 1, torch.from_numpy(ours)), vals)


@pytest.mark.parametrize("cap", ["0750", "0500", "0125"])
def test_mod_router_golden(cap):
    d = np.load(GOLDEN / f"mod_router_cap{cap}.npz")
    x, w, b = bf16_from_bits(d["x"]), bf16_from_bits(d["w"]), bf16_from_bits(d["b"])
    scores = F.linear(x, w, b).squeeze(-1)
    assert torch.equal(scores, torch.from_numpy(d["scores"]))
    L = x.shape[1]
    k = omod.router_k(L, float(d["capacity_ratio"]))
    assert k == d["indices"].shape[1]
    ours = omod.topk_desc_lowest_index(d["scores"], k)
    assert np.array_equal(ours, d["stable_order"])
    # torch.topk (what the reference calls) gives the same value sequence
    assert np.array_equal(np.take_along_axis(d["scores"], ours, 1),
                          np.take_along_axis(d["scores"], d["indices"], 1))
    # the reference mask marks exactly torch.topk's set
    assert np.array_equal(omod.mask_from_indices(d["indices"], L), d["mask"])


def test_residual_scatter_invariants():
    g = torch.Generator().manual_seed(9)
    h = torch.randn(2, 10, 4, generator=g)
    idx = torch.tensor([[7, 1, 3], [0, 9, 5]])
    y = torch.randn(2, 3, 4, generator=g)
    out = omod.residual_scatter(h, y, idx)
    for b in range(2):
        sel = set(idx[b].tolist())
        for s in range(10):
            if s in sel:
                j = idx[b].tolist().index(s)
                assert torch.equal(out[b, s], h[b, s] + y[b, j])
            else:
                assert torch.equal(out[b, s], h[b, s])
    rep = omod.replace_scatter(h, y, idx)
    assert torch.equal(rep[0, 7], y[0, 0]) and torch.equal(rep[0, 2], h[0, 2])
    gth = omod.gather(h, idx)
    assert torch.equal(gth[1, 1], h[1, 9])


# ---------------------------------------------------------------------------
# Backward of the fused ops
# ---------------------------------------------------------------------------
def _rms_bwd_golden():
    d = np.load(GOLDEN / "fused_ops_bwd_cpu.npz")
    return (bf16_from_bits(d["x"]), bf16_from_bits(d["w"]), bf16_from_bits(d["grad_out"]),
            float(d["eps"]), torch.from_numpy(d["rms_grad_x"]), torch.from_numpy(d["rms_grad_w"]))


def test_rms_norm_backward_golden():
    """The oracle equals the reference's _rms_norm_backward_pytorch on rows
    with mean(x^2) from ~0.04 to ~1600 and a clamped row."""
    x, w, go, eps, gx_ref, gw_ref = _rms_bwd_golden()
    gx, gw = ofo.rms_norm_backward(x, w, go, eps)
    assert torch.allclose(gx, gx_ref, rtol=1e-6, atol=1e-6)
    assert torch.allclose(gw, gw_ref, rtol=1e-6, atol=1e-5)
    assert gx.abs().max() <= 100.0 and (gx.abs() == 100.0).any()


def test_rms_norm_backward_autograd_where_exact():
    """grad_w is the exact derivative (autograd of F.rms_norm, fp64); grad_x
    is too on rows with mean(x^2) + eps = 1, where the reference's
    correction term loses nothing."""
    g = torch.Generator().manual_seed(21)
    rows, dim, eps = 6, 48, 1e-6
    x = torch.randn(rows, dim, generator=g, dtype=torch.float64)
    x = x / torch.sqrt(x.pow(2).mean(-1, keepdim=True)) * math.sqrt(1.0 - eps)
    w = torch.randn(dim, generator=g, dtype=torch.float64)
    go = torch.randn(rows, dim, generator=g, dtype=torch.float64)
    xa, wa = x.clone().requires_grad_(), w.clone().requires_grad_()
    F.rms_norm(xa, [dim], weight=wa, eps=eps).backward(go)
    gx, gw = ofo.rms_norm_backward(x.float(), w.float(), go.float(), eps)
    assert torch.allclose(gw.double(), wa.grad, rtol=1e-4, atol=1e-4)
    assert torch.allclose(gx.double(), xa.grad, rtol=1e-4, atol=1e-4)
    # and off unit RMS the written formula differs from the derivative
    x2 = x * 3.0
    xa2 = x2.clone().requires_grad_()
    F.rms_norm(xa2, [dim], weight=w, eps=eps).backward(go)
    gx2, _ = ofo.rms_norm_backward(x2.float(), w.float(), go.float(), eps)
    assert not torch.allclose(gx2.double(), xa2.grad, rtol=1e-2, atol=1e-2)


def test_swiglu_backward_autograd_and_clamp():
    g = torch.Generator().manual_seed(22)
    gate = torch.randn(5, 33, generator=g, dtype=torch.float64) * 3
    up = torch.randn(5, 33, generator=g, dtype=torch.float64)
    go = torch.randn(5, 33, generator=g, dtype=torch.float64)
    ga, ua = gate.clone().requires_grad_(), up.clone().requires_grad_()
    (F.silu(ga) * ua).backward(go)
    gg, gu = ofo.swiglu_backward(gate, up, go)
    # (the backward computes in fp32, as the reference's does)
    assert torch.allclose(gg, ga.grad, rtol=1e-5, atol=1e-6)
    assert torch.allclose(gu, ua.grad, rtol=1e-5, atol=1e-6)
    gg, gu = ofo.swiglu_backward(gate, up, go * 1e4)
    assert torch.allclose(gg, (ga.grad * 1e4).clamp(-100, 100), rtol=1e-5, atol=1e-4)
    assert gu.abs().max() == 100.0


def test_qk_norm_backward_autograd():
    g = torch.Generator().manual_seed(23)
    q = torch.randn(2, 3, 7, 16, generator=g, dtype=torch.float64)
    k = torch.randn(2, 1, 7, 16, generator=g, dtype=torch.float64) * 4
    gq = torch.randn_like(q)
    gk = torch.randn_like(k)
    qa, ka = q.clone().requires_grad_(), k.clone().requires_grad_()
    qo, ko = ofo.qk_norm(qa, ka, 2.5, 0.6)
    torch.autograd.backward([qo, ko], [gq, gk])
    dq, dk = ofo.qk_norm_backward(q, k, gq, gk, 2.5, 0.6)
    assert torch.allclose(dq, qa.grad, rtol=1e-5, atol=1e-6)
    assert torch.allclose(dk, ka.grad, rtol=1e-5, atol=1e-6)


def test_rope_backward_autograd():
    g = torch.Generator().manual_seed(24)
    x = torch.randn(2, 3, 11, 16, generator=g, dtype=torch.float64)
    go = torch.randn_like(x)
    cos, sin = ofo.rope_cache(16, 20)
    xa = x.clone().requires_grad_()
    ofo.rope(xa, cos.double(), sin.double()).backward(go)
    gx = ofo.rope_backward(go, cos, sin)
    assert torch.allclose(gx, xa.grad, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(2, 4, 1, 9, 8), (1, 4, 2, 13, 6), (1, 2, 2, 5, 4)])
def test_attention_backward_autograd(causal, shape):
    """The split-K restatement (explicit P, D = rowsum(dO * O), head sums
    over the GQA group) against autograd through the forward oracle, which
    expands K/V by repeat_interleave: a wrong head mapping, a missing scale
    or D taken from the wrong side fails here."""
    B, Hq, Hkv, S, hd = shape
    g = torch.Generator().manual_seed(S * hd + causal)
    q, k, v = (torch.randn(B, h, S, hd, generator=g, dtype=torch.float64).requires_grad_()
               for h in (Hq, Hkv, Hkv))
    go = torch.randn(B, Hq, S, hd, generator=g, dtype=torch.float64)
    occ.attention_key_padding(q, k, v, causal=causal).backward(go)
    dq, dk, dv = occ.attention_backward(q.detach(), k.detach(), v.detach(), go, causal=causal)
    for got, ref in ((dq, q.grad), (dk, k.grad), (dv, v.grad)):
        assert torch.allclose(got, ref, rtol=1e-10, atol=1e-12)
    # a non-default scale, and causal row 0 whose only key is itself: dq = 0 there
    q2 = q.detach().clone().requires_grad_()
    occ.attention_key_padding(q2, k.detach(), v.detach(), causal=causal, scale=0.3).backward(go)
    dq2, _, _ = occ.attention_backward(q2.detach(), k.detach(), v.detach(), go, causal=causal, scale=0.3)
    assert torch.allclose(dq2, q2.grad, rtol=1e-10, atol=1e-12)
    if causal:
        assert dq[:, :, 0].abs().max() < 1e-12


def test_chunked_cross_entropy_autograd():
    """The restated chunked CE against autograd of F.cross_entropy (fp64) with
    ignore_index, including out-of-range targets (then the whole target
    vector is clamped, ignore entries included, fused_ops.py:1407-1422), the
    same targets without the out-of-range ones (ignore entries stay ignored)
    and the all-ignored case (loss 0, zero gradients)."""
    g = torch.Generator().manual_seed(11)
    h = torch.randn(3, 7, 16, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(50, 16, generator=g, dtype=torch.float64, requires_grad=True)
    t = torch.randint(0, 50, (3, 7), generator=g)
    t[0, 1] = -100
    t[2, 3] = -100
    t[1, 2] = 57   # clamped to 49
    t[1, 4] = -7   # clamped to 0
    for tt, tc in ((t, t.clamp(0, 49)),
                   (torch.where((t < 0) & (t != -100), 0, torch.where(t > 49, 49, t)),) * 2):
        h.grad = w.grad = None
        ref = F.cross_entropy((h.reshape(-1, 16) @ w.t()), tc.reshape(-1), ignore_index=-100)
        ref.backward(torch.tensor(0.7, dtype=torch.float64))
        loss, gh, gw = ofo.chunked_cross_entropy(h.detach(), w.detach(), tt, grad_output=0.7)
        assert torch.allclose(loss, ref.detach(), rtol=1e-12)
        assert torch.allclose(gh, h.grad, rtol=1e-10, atol=1e-13)
        assert torch.allclose(gw, w.grad, rtol=1e-10, atol=1e-13)
    loss0, gh0, gw0 = ofo.chunked_cross_entropy(h.detach(), w.detach(), torch.full((3, 7), -100))
    assert loss0 == 0 and gh0.abs().max() == 0 and gw0.abs().max() == 0


def test_token_losses_match_cross_entropy_none():
    """token_losses_from_hidden = F.cross_entropy(reduction='none') (fp64)
    with ignore_index; with an out-of-range target the reference clamps the
    ignore entries too, so they turn into target-0 losses."""
    g = torch.Generator().manual_seed(12)
    h = torch.randn(2, 5, 8, generator=g, dtype=torch.float64)
    w = torch.randn(30, 8, generator=g, dtype=torch.float64)
    t = torch.randint(0, 30, (2, 5), generator=g)
    t[0, 0] = -100
    ref = F.cross_entropy(h.reshape(-1, 8) @ w.t(), t.reshape(-1), ignore_index=-100, reduction="none")
    assert torch.allclose(ofo.token_losses_from_hidden(h, w, t).reshape(-1), ref, rtol=1e-12)
    t[1, 1] = 31
    got = ofo.token_losses_from_hidden(h, w, t).reshape(-1)
    tc = t.clamp(0, 29).reshape(-1)
    ref = F.cross_entropy(h.reshape(-1, 8) @ w.t(), tc, reduction="none")
    assert torch.allclose(got, ref, rtol=1e-12) and got[0] > 0
