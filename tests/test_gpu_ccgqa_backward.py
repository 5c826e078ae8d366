"""GPU parity of the CCGQA training path: CCGQAPrepFunction (the prep
kernel's forward with hydra_ccgqa_prep_bwd and the conv GEMMs behind it)
and the whole CCGQAAttention module backward, against torch autograd
through the oracle's forward (oracle.ccgqa.prep / forward, restating
attention.py:201-331) in fp64 on the CPU.  Tolerance (normwise max-rel-err
of every gradient): fp32 1e-4 (fp32 GEMM and kernel sums over up to 16K
tokens against fp64), bf16 5e-2 (bf16 gradients through bf16 GEMMs against
fp64 autograd of the same bf16-valued inputs)."""
from __future__ import annotations

import pytest
import torch

from conftest import max_rel_err
from oracle import ccgqa as occ

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 5e-2}
CONV_NAMES = ("q_conv.conv1.weight", "q_conv.conv2.weight", "k_conv.conv1.weight",
              "k_conv.conv2.weight")

CASES = [
    # config 3's heads (4 q / 1 kv of 64): QK-mean of means, MFMA prep path
    dict(dim=1024, n_heads=4, n_kv_heads=1, compression_factor=4, B=1, S=128),
    # one q head per kv head (QK-mean (q0 + k0) / 2), head_dim 32
    dict(dim=512, n_heads=4, n_kv_heads=4, compression_factor=4, B=2, S=96),
    # head_dim 16, GQA 2, ragged length
    dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, B=2, S=77),
    # no convs
    dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, B=1, S=40, use_convs=False),
    # every optional feature off
    dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, B=1, S=40, use_qk_norm=False,
         use_rope=False, use_value_shift=False, use_qk_mean=False),
]


def _setup(case, dtype, seed):
    case = dict(case)
    B, S = case.pop("B"), case.pop("S")
    cfg = occ.CCGQAConfig(max_seq_len=max(256, S), **case)
    g = torch.Generator().manual_seed(seed)
    params = occ.init_params(cfg, g, std=0.1, temperature=1.7)
    params = {k: v.to(dtype) for k, v in params.items()}
    return cfg, B, S, g, params


def _leaf64(t):
    return t.detach().double().requires_grad_(True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
def test_prep_backward(cuda, case, dtype):
    from hydra_amd.attention.backends.ccgqa.autograd import ccgqa_prep_train
    from hydra_amd.attention.backends.ccgqa.ops import prep_flags

    cfg, B, S, g, params = _setup(case, dtype, seed=41)
    L, K, hd = cfg.latent_dim, cfg.kv_dim, cfg.head_dim
    qkv = torch.randn(B, S, L + 2 * K, generator=g).to(dtype)
    gq = torch.randn(B, cfg.n_heads, S, hd, generator=g).to(dtype)
    gk = torch.randn(B, cfg.n_kv_heads, S, hd, generator=g).to(dtype)
    gv = torch.randn(B, cfg.n_kv_heads, S, hd, generator=g).to(dtype)
    cos, sin = occ.fused_ops.rope_cache(hd, S)

    # oracle: autograd through the prep in fp64
    p64 = {k: _leaf64(v) for k, v in params.items()}
    x64 = _leaf64(qkv)
    q, k, v = occ.prep(p64, x64, cfg, cos.double(), sin.double())
    ((q * gq.double()).sum() + (k * gk.double()).sum() + (v * gv.double()).sum()).backward()

    # device
    flags = prep_flags(cfg.use_convs, cfg.use_qk_mean, cfg.use_value_shift, cfg.use_qk_norm, cfg.use_rope)
    dp = {k: v.to(cuda).requires_grad_(True) for k, v in params.items()}
    xd = qkv.to(cuda).requires_grad_(True)
    w = [dp.get(n) for n in CONV_NAMES]
    qd, kd, vd = ccgqa_prep_train(xd, cfg.n_heads, cfg.n_kv_heads, hd, flags, *w,
                                  temperature=dp["key_temperature"] if cfg.use_qk_norm else None,
                                  cos=cos.to(cuda) if cfg.use_rope else None,
                                  sin=sin.to(cuda) if cfg.use_rope else None)
    for got, want in zip((qd, kd, vd), (q, k, v)):  # the forward is the inference kernel's
        assert max_rel_err(got.cpu(), want) < (1e-5 if dtype == torch.float32 else 2e-2)
    torch.autograd.backward((qd, kd, vd), (gq.to(cuda), gk.to(cuda), gv.to(cuda)))
    tol = TOL[dtype]
    assert max_rel_err(xd.grad.cpu(), x64.grad) < tol
    for n in CONV_NAMES:
        if n in params:
            assert max_rel_err(dp[n].grad.cpu(), p64[n].grad) < tol, n
    if cfg.use_qk_norm:
        assert max_rel_err(dp["key_temperature"].grad.cpu(), p64["key_temperature"].grad) < tol
    # no gradient path the oracle does not have
    assert dp["qkv_proj.weight"].grad is None


MODULE_CASES = CASES[:3] + [
    # config 3's module (dim 1024, 4/1 heads of 64) at B 2 x S 1024
    dict(dim=1024, n_heads=4, n_kv_heads=1, compression_factor=4, B=2, S=1024),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", MODULE_CASES, ids=[str(i) for i in range(len(MODULE_CASES))])
def test_module_backward(cuda, case, dtype):
    """CCGQAAttention forward + backward (training path) against fp64
    autograd through oracle.ccgqa.forward: x and every parameter."""
    from hydra_amd.attention import CCGQAAttention

    cfg, B, S, g, params = _setup(case, dtype, seed=43)
    x = torch.randn(B, S, cfg.dim, generator=g).to(dtype)
    gout = torch.randn(B, S, cfg.dim, generator=g).to(dtype)

    p64 = {k: _leaf64(v) for k, v in params.items()}
    x64 = _leaf64(x)
    out = occ.forward(p64, x64, cfg)
    (out * gout.double()).sum().backward()

    m = CCGQAAttention(dim=cfg.dim, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                       compression_factor=cfg.compression_factor, max_seq_len=cfg.max_seq_len)
    m.load_state_dict(params)
    m = m.to(device=cuda, dtype=dtype).train()
    xd = x.to(cuda).requires_grad_(True)
    od = m(xd)
    assert max_rel_err(od.detach().cpu(), out) < (1e-5 if dtype == torch.float32 else 2e-2)
    od.backward(gout.to(cuda))
    tol = TOL[dtype]
    assert max_rel_err(xd.grad.cpu(), x64.grad) < tol
    for n, prm in m.named_parameters():
        assert prm.grad is not None, n
        assert max_rel_err(prm.grad.cpu(), p64[n].grad) < tol, n


def test_module_train_step_reduces_loss(cuda):
    """A few SGD steps through the module's backward reduce a regression
    loss (the gradients point downhill end to end)."""
    from hydra_amd.attention import CCGQAAttention

    torch.manual_seed(0)
    m = CCGQAAttention(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, max_seq_len=128).to(cuda)
    x = torch.randn(2, 64, 256, device=cuda)
    target = torch.randn(2, 64, 256, device=cuda) * 0.1
    opt = torch.optim.SGD(m.parameters(), lr=0.5)
    losses = []
    for _ in range(5):
        opt.zero_grad()
        loss = ((m(x) - target) ** 2).mean()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0]


@pytest.mark.parametrize("semantics", ["reference", "key_padding"])
def test_module_backward_with_mask(cuda, monkeypatch, semantics):
    """CCGQAAttention with a padding mask trains: forward + backward against
    fp64 autograd through oracle.ccgqa.forward with the same mask, in the
    reference's literal semantics (attention.py:268-299) and the key-padding
    reading."""
    from hydra_amd.attention import CCGQAAttention

    monkeypatch.setenv("HYDRA_CCGQA_MASK_SEMANTICS", semantics)
    case = dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, B=2, S=48)
    cfg, B, S, g, params = _setup(case, torch.float32, seed=44)
    x = torch.randn(B, S, cfg.dim, generator=g)
    gout = torch.randn(B, S, cfg.dim, generator=g)
    mask = (torch.rand(B, S, generator=g) > 0.3).long()
    mask[:, 0] = 1
    mask[:, S // 2] = 0
    p64 = {k: _leaf64(v) for k, v in params.items()}
    x64 = _leaf64(x)
    if semantics == "reference":
        out = occ.forward(p64, x64, cfg, mask=mask)
    else:
        qkv = torch.nn.functional.linear(x64, p64["qkv_proj.weight"])
        q, k, v = occ.prep(p64, qkv, cfg)
        o = occ.attention_key_padding(q, k, v, causal=True, mask=mask)
        o = o.transpose(1, 2).reshape(B, S, cfg.latent_dim)
        out = torch.nn.functional.linear(o, p64["o_proj.weight"])
    (out * gout.double()).sum().backward()

    m = CCGQAAttention(dim=cfg.dim, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                       compression_factor=cfg.compression_factor, max_seq_len=cfg.max_seq_len)
    m.load_state_dict(params)
    m = m.to(cuda).train()
    xd = x.to(cuda).requires_grad_(True)
    od = m(xd, mask=mask.to(cuda))
    assert max_rel_err(od.detach().cpu(), out) < 1e-5
    od.backward(gout.to(cuda))
    assert max_rel_err(xd.grad.cpu(), x64.grad) < 1e-4
    for n, prm in m.named_parameters():
        assert prm.grad is not None, n
        assert max_rel_err(prm.grad.cpu(), p64[n].grad) < 1e-4, n


def test_module_eval_under_grad_uses_inference_kernels(cuda):
    """model.eval() with parameters that require grad, outside no_grad:
    the forward runs the inference kernels (the same bits as under
    no_grad), and a backward recomputes the training path, giving the
    gradients train() mode gives for the same input."""
    from hydra_amd.attention import CCGQAAttention

    torch.manual_seed(7)
    m = CCGQAAttention(dim=1024, n_heads=4, n_kv_heads=1, compression_factor=4,
                       max_seq_len=256).to(cuda, torch.bfloat16)
    with torch.no_grad():
        m.key_temperature.fill_(1.0)
    x = torch.randn(2, 256, 1024, device=cuda, dtype=torch.bfloat16)
    gout = torch.randn(2, 256, 1024, device=cuda, dtype=torch.bfloat16)
    m.eval()
    with torch.no_grad():
        want = m(x)
    got = m(x)
    assert got.requires_grad and torch.equal(got.detach(), want)
    got.backward(gout)
    eval_grads = {n: p.grad.clone() for n, p in m.named_parameters()}
    m.zero_grad(set_to_none=True)
    m.train()
    out = m(x)
    assert max_rel_err(out.detach().float().cpu(), want.float().cpu()) < 2e-2
    out.backward(gout)
    for n, p in m.named_parameters():
        assert torch.equal(p.grad, eval_grads[n]), n


@pytest.mark.parametrize("ks", [2, 5])
def test_module_backward_conv_kernel_sizes(cuda, ks):
    """The training path with conv_kernel_size != 3 (the im2col columns take
    ks taps): forward + backward against fp64 autograd through
    oracle.ccgqa.forward."""
    from hydra_amd.attention import CCGQAAttention

    case = dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, B=2, S=40,
                conv_kernel_size=ks)
    cfg, B, S, g, params = _setup(case, torch.float32, seed=45 + ks)
    x = torch.randn(B, S, cfg.dim, generator=g)
    gout = torch.randn(B, S, cfg.dim, generator=g)
    p64 = {k: _leaf64(v) for k, v in params.items()}
    x64 = _leaf64(x)
    out = occ.forward(p64, x64, cfg)
    (out * gout.double()).sum().backward()
    m = CCGQAAttention(dim=cfg.dim, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                       compression_factor=cfg.compression_factor, max_seq_len=cfg.max_seq_len,
                       conv_kernel_size=ks)
    m.load_state_dict(params)
    m = m.to(cuda).train()
    xd = x.to(cuda).requires_grad_(True)
    od = m(xd)
    assert max_rel_err(od.detach().cpu(), out) < 1e-5
    od.backward(gout.to(cuda))
    assert max_rel_err(xd.grad.cpu(), x64.grad) < 1e-4
    for n, prm in m.named_parameters():
        assert max_rel_err(prm.grad.cpu(), p64[n].grad) < 1e-4, n
