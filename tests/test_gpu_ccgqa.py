"""GPU parity of the CCGQA forward: the fused prep kernel against the
oracle's prep, and the whole CCGQAAttention module against the golden
vectors written by running the reference module, and against the oracle at
the benchmark configurations.  fp32 bar 1e-5, bf16 bar 2e-2 (normwise)."""
from __future__ import annotations

import pytest
import torch

from conftest import GOLDEN, max_rel_err
from oracle import ccgqa as occ
from test_oracle_pins import load_ccgqa_golden

pytestmark = pytest.mark.gpu

GOLDEN_CCGQA = sorted(GOLDEN.glob("ccgqa_*.npz"))


def _module(cfg: occ.CCGQAConfig, params: dict, device, dtype):
    from hydra_amd.attention import CCGQAAttention

    m = CCGQAAttention(dim=cfg.dim, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                       compression_factor=cfg.compression_factor, max_seq_len=cfg.max_seq_len,
                       use_rope=cfg.use_rope, use_qk_norm=cfg.use_qk_norm, use_convs=cfg.use_convs,
                       use_qk_mean=cfg.use_qk_mean, use_value_shift=cfg.use_value_shift)
    m.load_state_dict(params)
    return m.to(device=device, dtype=dtype).eval()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("path", GOLDEN_CCGQA, ids=[p.stem for p in GOLDEN_CCGQA])
def test_module_matches_reference_golden(cuda, path, dtype):
    cfg, params, x, mask, out = load_ccgqa_golden(path)
    m = _module(cfg, params, cuda, dtype)
    with torch.no_grad():
        got = m(x.to(cuda, dtype), mask=None if mask is None else mask.to(cuda)).float().cpu()
    assert max_rel_err(got, out) < (1e-5 if dtype == torch.float32 else 2e-2)


PREP_CASES = [
    # dim, Hq, Hkv, C, B, S, flags
    dict(dim=1024, n_heads=4, n_kv_heads=1, compression_factor=4, B=2, S=300),
    dict(dim=512, n_heads=8, n_kv_heads=2, compression_factor=4, B=2, S=512),
    dict(dim=256, n_heads=4, n_kv_heads=4, compression_factor=2, B=1, S=77),
    dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, B=1, S=9, use_convs=False),
    dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, B=1, S=40, use_qk_norm=False,
         use_rope=False, use_value_shift=False, use_qk_mean=False),
    # head_dim 128 on the MFMA path (4 m-tiles per head), GQA 2
    dict(dim=2048, n_heads=4, n_kv_heads=2, compression_factor=4, B=1, S=200),
    # head_dim 32, one q head per kv head (QK-mean (q0 + k0) / 2), no convs
    dict(dim=512, n_heads=4, n_kv_heads=4, compression_factor=4, B=2, S=96, use_convs=False),
    # config 5's layout: latent 448, 28 q / 4 kv heads of 16 (MFMA path, two
    # heads per conv m-tile, block-diagonal conv1)
    dict(dim=1792, n_heads=28, n_kv_heads=4, compression_factor=4, B=1, S=264),
    # head_dim 16 with a ragged last tile
    dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, B=2, S=77),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", PREP_CASES, ids=[str(i) for i in range(len(PREP_CASES))])
def test_prep_kernel(cuda, case, dtype):
    from hydra_amd.attention.backends.ccgqa.ops import ccgqa_prep, prep_flags

    case = dict(case)
    B, S = case.pop("B"), case.pop("S")
    cfg = occ.CCGQAConfig(max_seq_len=1024, **case)
    g = torch.Generator().manual_seed(31)
    params = occ.init_params(cfg, g, temperature=1.0)
    params = {k: v.to(dtype) for k, v in params.items()}
    qkv = torch.randn(B, S, cfg.latent_dim + 2 * cfg.kv_dim, generator=g).to(dtype)
    ref = occ.prep({k: v.float() for k, v in params.items()}, qkv.float(), cfg)
    cos, sin = occ.fused_ops.rope_cache(cfg.head_dim, S)
    conv = [params.get(n) for n in ("q_conv.conv1.weight", "q_conv.conv2.weight",
                                    "k_conv.conv1.weight", "k_conv.conv2.weight")]
    flags = prep_flags(cfg.use_convs, cfg.use_qk_mean, cfg.use_value_shift, cfg.use_qk_norm, cfg.use_rope)
    q, k, v = ccgqa_prep(qkv.to(cuda), cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, flags,
                         *[None if w is None else w.to(cuda) for w in conv],
                         temperature=params["key_temperature"].to(cuda),
                         cos=cos.to(cuda), sin=sin.to(cuda))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for got, want in zip((q, k, v), ref):
        assert max_rel_err(got.cpu(), want) < tol
    assert torch.equal(v.cpu().float(), ref[2].to(dtype).float())  # the value shift is a copy
    # V^T output layout: the same values, transposed in memory
    from hydra_amd._lib import CCGQA_V_TRANSPOSED

    if S % 8 == 0 or dtype == torch.float32:
        q2, k2, v2 = ccgqa_prep(qkv.to(cuda), cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                flags | CCGQA_V_TRANSPOSED,
                                *[None if w is None else w.to(cuda) for w in conv],
                                temperature=params["key_temperature"].to(cuda),
                                cos=cos.to(cuda), sin=sin.to(cuda))
        assert v2.stride(-2) == 1
        assert torch.equal(v2.cpu(), v.cpu())
        assert torch.equal(q2.cpu(), q.cpu()) and torch.equal(k2.cpu(), k.cpu())
    # MFMA-tiled conv weights: the same operands in a different memory order
    from hydra_amd._lib import CCGQA_W_TILED
    from hydra_amd.attention.backends.ccgqa.ops import tiled_weights_ok

    if cfg.use_convs and tiled_weights_ok(cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, dtype):
        q3, k3, v3 = ccgqa_prep(qkv.to(cuda), cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                flags | CCGQA_W_TILED, *[w.to(cuda) for w in conv],
                                temperature=params["key_temperature"].to(cuda),
                                cos=cos.to(cuda), sin=sin.to(cuda))
        assert torch.equal(q3.cpu(), q.cpu()) and torch.equal(k3.cpu(), k.cpu())
        assert torch.equal(v3.cpu(), v.cpu())
    # no tile's epilogue gave up waiting for its QK-mean terms
    from hydra_amd import _lib

    assert _lib.prep_faults() == 0


def _bench_case(dim, n_heads, n_kv_heads, B, S, dtype, temperature, seed):
    cfg = occ.CCGQAConfig(dim=dim, n_heads=n_heads, n_kv_heads=n_kv_heads, compression_factor=4,
                          max_seq_len=max(S, 8))
    g = torch.Generator().manual_seed(seed)
    params = {k: v.to(dtype).float() for k, v in occ.init_params(cfg, g, temperature=temperature).items()}
    x = torch.randn(B, S, dim, generator=g).to(dtype).float()
    return cfg, params, x


def test_c1_debug_shape_fp32(cuda):
    """Config 1's attention: dim 512, 8/2 heads, C=4 (hd 16), B2 x S512, fp32."""
    cfg, params, x = _bench_case(512, 8, 2, 2, 512, torch.float32, None, 41)
    want = occ.forward(params, x, cfg)
    m = _module(cfg, params, cuda, torch.float32)
    with torch.no_grad():
        got = m(x.to(cuda)).cpu()
    assert max_rel_err(got, want) < 1e-5


def test_c3_shape_bf16(cuda):
    """Config 3: dim 1024, 4/1 heads (hd 64), C=4, tau 1.0, B4 x S4096, bf16."""
    cfg, params, x = _bench_case(1024, 4, 1, 4, 4096, torch.bfloat16, 1.0, 42)
    want = occ.forward(params, x, cfg)
    m = _module(cfg, params, cuda, torch.bfloat16)
    with torch.no_grad():
        got = m(x.to(cuda, torch.bfloat16)).float().cpu()
    assert max_rel_err(got, want) < 2e-2


def test_standalone_conv_sequence(cuda):
    from hydra_amd.attention.backends.ccgqa.kernels.fused_conv import OptimizedConvSequence

    g = torch.Generator().manual_seed(43)
    mod = OptimizedConvSequence(64, 4, 1, 3)
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.1)
    x = torch.randn(2, 50, 64, generator=g)
    want = occ.causal_conv_seq(x, mod.conv1.weight.detach(), mod.conv2.weight.detach(), 4)
    got = mod.to(cuda)(x.to(cuda)).detach().cpu()
    assert max_rel_err(got, want) < 1e-5


def test_prep_generic_kernel_fallback(cuda, monkeypatch):
    """The one-thread-per-output VALU prep kernel (forced; otherwise taken
    only by layouts the other kernels reject) against the oracle, fp32."""
    from hydra_amd.attention.backends.ccgqa.ops import ccgqa_prep, prep_flags

    monkeypatch.setenv("HYDRA_PREP_GENERIC", "1")
    cfg = occ.CCGQAConfig(dim=512, n_heads=8, n_kv_heads=2, compression_factor=4, max_seq_len=256)
    g = torch.Generator().manual_seed(32)
    params = occ.init_params(cfg, g, temperature=1.0)
    qkv = torch.randn(2, 70, cfg.latent_dim + 2 * cfg.kv_dim, generator=g)
    ref = occ.prep(params, qkv, cfg)
    cos, sin = occ.fused_ops.rope_cache(cfg.head_dim, 70)
    conv = [params[n].to(cuda) for n in ("q_conv.conv1.weight", "q_conv.conv2.weight",
                                          "k_conv.conv1.weight", "k_conv.conv2.weight")]
    q, k, v = ccgqa_prep(qkv.to(cuda), cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                         prep_flags(True, True, True, True, True), *conv,
                         temperature=params["key_temperature"].to(cuda), cos=cos.to(cuda), sin=sin.to(cuda))
    for got, want in zip((q, k, v), ref):
        assert max_rel_err(got.cpu(), want) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ks", [1, 2, 5])
def test_module_conv_kernel_sizes(cuda, dtype, ks):
    """conv_kernel_size other than 3 (attention.py:132-145 builds both conv
    sequences with it; fused_conv.py:52-57 pads by k-1): the module against
    the oracle's forward, in fp32 and bf16, and the standalone conv
    sequence against oracle.causal_conv_seq."""
    from hydra_amd.attention import CCGQAAttention
    from hydra_amd.attention.backends.ccgqa.kernels.fused_conv import OptimizedConvSequence

    cfg = occ.CCGQAConfig(dim=512, n_heads=4, n_kv_heads=2, compression_factor=4, max_seq_len=128,
                          conv_kernel_size=ks)
    g = torch.Generator().manual_seed(50 + ks)
    params = {k: v.to(dtype) for k, v in occ.init_params(cfg, g, std=0.05, temperature=2.0).items()}
    x = torch.randn(2, 96, 512, generator=g).to(dtype)
    want = occ.forward({k: v.float() for k, v in params.items()}, x.float(), cfg)
    m = CCGQAAttention(dim=512, n_heads=4, n_kv_heads=2, compression_factor=4, max_seq_len=128,
                       conv_kernel_size=ks)
    m.load_state_dict(params)
    with torch.no_grad():
        got = m.to(cuda, dtype)(x.to(cuda)).float().cpu()
    assert max_rel_err(got, want) < (1e-5 if dtype == torch.float32 else 2e-2)
    seq = OptimizedConvSequence(128, 4, 1, ks).to(cuda, dtype)
    seq.load_state_dict({"conv1.weight": params["q_conv.conv1.weight"],
                         "conv2.weight": params["q_conv.conv2.weight"]})
    xs = torch.randn(2, 70, 128, generator=g).to(dtype)
    with torch.no_grad():
        ys = seq(xs.to(cuda)).float().cpu()
    ref = occ.causal_conv_seq(xs.float(), params["q_conv.conv1.weight"].float(),
                              params["q_conv.conv2.weight"].float(), 4)
    assert max_rel_err(ys, ref) < (1e-5 if dtype == torch.float32 else 2e-2)
