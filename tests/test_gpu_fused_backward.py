"""GPU parity of the fused ops' backward (RMSNorm, SwiGLU, QK-norm, RoPE)
against the oracle's restatement of the reference's PyTorch backward on the
same inputs (the oracle itself is pinned by autograd and by the reference's
own vectors in tests/test_oracle_pins.py).

Both sides compute in fp32 and round once, so they differ only by summation
order: normwise max-rel-err < 1e-5 for fp32, < 1e-2 for bf16 (a bf16 ulp
is 2^-8 relative; an order change can move a rounding by one ulp).  Clamps
to +-100 are checked exactly."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN, bf16_from_bits, max_rel_err
from oracle import fused_ops as ofo

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def _gen(seed=0):
    return torch.Generator().manual_seed(seed)


# --------------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(4, 512, 1792), (2, 128, 768), (1, 1, 64), (3, 7, 80), (2, 256, 768),
                                   (5, 13), (9, 2056), (300, 32)])
def test_rms_norm_backward(cuda, dtype, shape):
    from hydra_amd.kernels.fused_ops import _RMSNormFunction

    g = _gen(sum(shape))
    dim = shape[-1]
    # rows with mean(x^2) far from 1, where the reference's grad_x formula
    # and the exact derivative part ways
    x = (torch.randn(*shape, generator=g) * 2.5).to(dtype)
    w = torch.randn(dim, generator=g).to(dtype)
    go = torch.randn(*shape, generator=g).to(dtype)
    xd, wd = x.to(cuda).requires_grad_(), w.to(cuda).requires_grad_()
    y = _RMSNormFunction.apply(xd, wd, 1e-6)
    y.backward(go.to(cuda))
    gx_ref, gw_ref = ofo.rms_norm_backward(x, w, go, 1e-6)
    assert xd.grad.dtype == dtype and wd.grad.dtype == dtype
    assert max_rel_err(xd.grad.cpu(), gx_ref) < TOL[dtype]
    tol_w = 1e-4 if dtype == torch.float32 else 1e-2  # sum over rows in another order
    assert max_rel_err(wd.grad.cpu(), gw_ref) < tol_w


def test_rms_norm_backward_reference_vectors(cuda):
    """The reference's own _rms_norm_backward_pytorch outputs (written by
    tests/golden/make_golden.py), on bf16 inputs computed in fp32."""
    from hydra_amd.kernels.fused_ops import _RMSNormFunction

    d = np.load(GOLDEN / "fused_ops_bwd_cpu.npz")
    x, w, go = bf16_from_bits(d["x"]), bf16_from_bits(d["w"]), bf16_from_bits(d["grad_out"])
    xd, wd = x.to(cuda).requires_grad_(), w.to(cuda).requires_grad_()
    _RMSNormFunction.apply(xd, wd, float(d["eps"])).backward(go.to(cuda))
    assert max_rel_err(xd.grad.cpu(), torch.from_numpy(d["rms_grad_x"])) < 1e-5
    assert max_rel_err(wd.grad.cpu(), torch.from_numpy(d["rms_grad_w"])) < 1e-5


def test_rms_norm_backward_clamp_and_determinism(cuda):
    """test_fused_backward_kernels.py:132-153: x = 1000, w = 10, g = 100 drive
    both gradients into the +-100 clamp; a repeated call is bit-identical."""
    from hydra_amd.kernels.fused_ops import _RMSNormFunction

    x = torch.full((4, 256, 768), 1000.0, device=cuda, dtype=torch.bfloat16)
    w = torch.full((768,), 10.0, device=cuda, dtype=torch.bfloat16)
    go = torch.full_like(x, 100.0)
    grads = []
    for _ in range(2):
        xd, wd = x.clone().requires_grad_(), w.clone().requires_grad_()
        _RMSNormFunction.apply(xd, wd, 1e-6).backward(go)
        grads.append((xd.grad, wd.grad))
        assert xd.grad.abs().max() <= 100.0 and wd.grad.abs().max() <= 100.0
    assert torch.equal(wd.grad.cpu(), torch.full((768,), 100.0, dtype=torch.bfloat16))
    g = _gen(5)
    xr = torch.randn(512, 768, generator=g).to(torch.bfloat16).to(cuda)
    gr = torch.randn(512, 768, generator=g).to(torch.bfloat16).to(cuda)
    outs = []
    for _ in range(2):
        xd, wd = xr.clone().requires_grad_(), w.clone().requires_grad_()
        _RMSNormFunction.apply(xd, wd, 1e-6).backward(gr)
        outs.append((xd.grad.clone(), wd.grad.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_rms_norm_backward_strided_rows(cuda):
    from hydra_amd.kernels import fused_rms_norm

    g = _gen(6)
    base = torch.randn(64, 1024, generator=g).to(torch.bfloat16)
    w = torch.randn(512, generator=g).to(torch.bfloat16)
    go = torch.randn(64, 512, generator=g).to(torch.bfloat16)
    bd = base.to(cuda).requires_grad_()
    wd = w.to(cuda).requires_grad_()
    fused_rms_norm(bd[:, 256:768], wd).backward(go.to(cuda))
    gx_ref, gw_ref = ofo.rms_norm_backward(base[:, 256:768], w, go, 1e-6)
    assert max_rel_err(bd.grad[:, 256:768].cpu(), gx_ref) < 1e-2
    assert torch.count_nonzero(bd.grad[:, :256]) == 0 and torch.count_nonzero(bd.grad[:, 768:]) == 0
    assert max_rel_err(wd.grad.cpu(), gw_ref) < 1e-2


# ---------------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,hidden", [(16384, 2048), (7, 40), (3, 13), (1, 8)])
def test_swiglu_backward_through_gate_up(cuda, dtype, rows, hidden):
    """gate/up are the halves of one gate_up tensor (the reference's caller,
    common.py:224-230); its gradient is the two halves' gradients."""
    from hydra_amd.kernels import fused_swiglu

    g = _gen(rows + hidden)
    gu = (torch.randn(rows, 2 * hidden, generator=g) * 2).to(dtype)
    go = torch.randn(rows, hidden, generator=g).to(dtype)
    gud = gu.to(cuda).requires_grad_()
    gate, up = gud.chunk(2, -1)
    fused_swiglu(gate, up).backward(go.to(cuda))
    gg_ref, gu_ref = ofo.swiglu_backward(gu[:, :hidden], gu[:, hidden:], go)
    assert max_rel_err(gud.grad[:, :hidden].cpu(), gg_ref) < TOL[dtype]
    assert max_rel_err(gud.grad[:, hidden:].cpu(), gu_ref) < TOL[dtype]


def test_swiglu_backward_clamp(cuda):
    from hydra_amd.kernels import fused_swiglu

    g = _gen(8)
    gate = (torch.randn(64, 96, generator=g) * 4).to(cuda).requires_grad_()
    up = (torch.randn(64, 96, generator=g) * 4).to(cuda).requires_grad_()
    go = torch.full((64, 96), 1e4, device=cuda)
    fused_swiglu(gate, up).backward(go)
    gg_ref, gu_ref = ofo.swiglu_backward(gate.detach().cpu(), up.detach().cpu(), go.cpu())
    assert gate.grad.abs().max() <= 100.0 and up.grad.abs().max() <= 100.0
    assert (gate.grad.abs() == 100.0).any()
    assert max_rel_err(gate.grad.cpu(), gg_ref) < 1e-5 and max_rel_err(up.grad.cpu(), gu_ref) < 1e-5


# --------------------------------------------------------------------- QK-norm
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shapes", [((4, 4, 512, 64), (4, 1, 512, 64)), ((2, 8, 64, 16), (2, 2, 64, 16)),
                                    ((1, 2, 33, 128), (1, 2, 33, 128)), ((2, 3, 5, 6), (2, 1, 5, 6))])
def test_qk_norm_backward(cuda, dtype, shapes):
    from hydra_amd.kernels import fused_qk_norm

    qs, ks = shapes
    g = _gen(qs[-1] + qs[2])
    q = (torch.randn(*qs, generator=g) * 3).to(dtype)
    k = torch.randn(*ks, generator=g).to(dtype)
    gq = torch.randn(*qs, generator=g).to(dtype)
    gk = torch.randn(*ks, generator=g).to(dtype)
    qd, kd = q.to(cuda).requires_grad_(), k.to(cuda).requires_grad_()
    qo, ko = fused_qk_norm(qd, kd, 8.0, 0.7)
    torch.autograd.backward([qo, ko], [gq.to(cuda), gk.to(cuda)])
    dq, dk = ofo.qk_norm_backward(q, k, gq, gk, 8.0, 0.7)
    assert max_rel_err(qd.grad.cpu(), dq) < TOL[dtype]
    assert max_rel_err(kd.grad.cpu(), dk) < TOL[dtype]


def test_qk_norm_backward_one_output_used(cuda):
    """Only q's output in the loss: k's upstream gradient is zero."""
    from hydra_amd.kernels import fused_qk_norm

    g = _gen(9)
    q = torch.randn(2, 4, 16, 32, generator=g)
    k = torch.randn(2, 2, 16, 32, generator=g)
    qd, kd = q.to(cuda).requires_grad_(), k.to(cuda).requires_grad_()
    qo, _ = fused_qk_norm(qd, kd, 2.0, 1.5)
    qo.sum().backward()
    dq, dk = ofo.qk_norm_backward(q, k, torch.ones_like(q), torch.zeros_like(k), 2.0, 1.5)
    assert max_rel_err(qd.grad.cpu(), dq) < 1e-5
    assert torch.count_nonzero(kd.grad) == 0


# ------------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(8, 12, 2048, 64), (2, 8, 512, 16), (1, 3, 17, 6), (2, 2, 5, 128)])
def test_rope_backward(cuda, dtype, shape):
    from hydra_amd.kernels import fused_rope

    B, H, S, D = shape
    g = _gen(S + D)
    x = torch.randn(*shape, generator=g).to(dtype)
    go = torch.randn(*shape, generator=g).to(dtype)
    cos, sin = ofo.rope_cache(D, S + 7)
    xd = x.to(cuda).requires_grad_()
    fused_rope(xd, cos.to(cuda), sin.to(cuda)).backward(go.to(cuda))
    ref = ofo.rope_backward(go, cos, sin)
    assert xd.grad.dtype == dtype
    assert max_rel_err(xd.grad.cpu(), ref) < (1e-6 if dtype == torch.float32 else 1e-2)


def test_rope_backward_strided_input_and_grad(cuda):
    """x a transposed view ([B,S,H,D] storage), the upstream gradient a
    non-contiguous view too."""
    from hydra_amd.kernels import fused_rope

    g = _gen(10)
    base = torch.randn(2, 40, 3, 32, generator=g)
    go_base = torch.randn(2, 3, 40, 64, generator=g)
    cos, sin = ofo.rope_cache(32, 40)
    bd = base.to(cuda).requires_grad_()
    x = bd.transpose(1, 2)
    go = go_base.to(cuda)[..., ::2]
    fused_rope(x, cos[0, 0].to(cuda), sin[0, 0].to(cuda)).backward(go)
    ref = ofo.rope_backward(go_base[..., ::2].contiguous(), cos, sin).transpose(1, 2)
    assert max_rel_err(bd.grad.cpu(), ref) < 1e-6
