"""GPU parity of the fused element ops (RMSNorm, RoPE, SwiGLU, QK-norm)
against the CPU oracle on the same seeded inputs.

Tolerances (normwise max-rel-err, conftest.max_rel_err): 1e-5 for fp32,
2e-2 for bf16/fp16 against the reference's CPU path; the kernels' own
arithmetic (fp32 inside, one rounding) is also checked against the oracle's
fp32-arithmetic variants at 1 ulp-level (8e-3 for bf16)."""
from __future__ import annotations

import pytest
import torch

from conftest import max_rel_err
from oracle import fused_ops as ofo

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _gen(seed=0):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(8, 2048, 768), (3, 5, 96), (7, 33), (2, 8192), (0, 64), (4, 1), (5, 2056)])
def test_rms_norm(cuda, dtype, shape):
    from hydra_amd.kernels import fused_rms_norm

    g = _gen(1)
    x = torch.randn(*shape, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], generator=g)).to(dtype)
    y = fused_rms_norm(x.to(cuda), w.to(cuda), 1e-6).cpu()
    assert y.dtype == dtype and y.shape == x.shape
    if x.numel() == 0:
        return
    ref = ofo.rms_norm(x.float(), w.float(), 1e-6)
    assert max_rel_err(y, ref) < TOL[dtype]
    assert max_rel_err(y, ofo.rms_norm_fp32(x, w, 1e-6)) < (1e-6 if dtype == torch.float32 else 8e-3)


def test_rms_norm_strided_rows(cuda):
    from hydra_amd.kernels import fused_rms_norm

    g = _gen(2)
    base = torch.randn(64, 2 * 512, generator=g).to(torch.bfloat16)
    x = base[:, 256:768]  # row stride 1024, width 512
    w = torch.ones(512, dtype=torch.bfloat16)
    y = fused_rms_norm(x.to(cuda), w.to(cuda)).cpu()
    assert max_rel_err(y, ofo.rms_norm(x.float(), w.float())) < 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(8, 12, 2048, 64), (2, 8, 512, 16), (1, 3, 17, 6), (2, 2, 5, 128), (1, 18, 33, 32)])
def test_rope(cuda, dtype, shape):
    from hydra_amd.kernels import fused_rope

    B, H, S, D = shape
    g = _gen(3)
    x = torch.randn(*shape, generator=g).to(dtype)
    cos, sin = ofo.rope_cache(D, S + 7)
    y = fused_rope(x.to(cuda), cos.to(cuda), sin.to(cuda)).cpu()
    assert y.dtype == dtype and y.shape == x.shape and y.is_contiguous()
    ref = ofo.rope(x.float(), cos, sin)
    assert max_rel_err(y, ref) < TOL[dtype]


def test_rope_many_batch_head_groups(cuda):
    """B x (head groups) past 65535: the launch spreads them over grid y and z."""
    from hydra_amd.kernels import fused_rope

    g = _gen(11)
    x = torch.randn(65600, 6, 2, 64, generator=g).to(torch.bfloat16)
    cos, sin = ofo.rope_cache(64, 2)
    y = fused_rope(x.to(cuda), cos.to(cuda), sin.to(cuda)).cpu()
    assert max_rel_err(y, ofo.rope(x.float(), cos, sin)) < TOL[torch.bfloat16]


def test_rope_cache_row_stride_not_vector_aligned(cuda):
    """cos/sin rows 35 elements apart: the per-element cos/sin loads."""
    from hydra_amd.kernels import fused_rope

    g = _gen(5)
    x = torch.randn(2, 12, 40, 64, generator=g).to(torch.bfloat16)
    cos, sin = ofo.rope_cache(64, 40)
    cw = torch.zeros(40, 35)
    sw = torch.zeros(40, 35)
    cw[:, :32], sw[:, :32] = cos[0, 0], sin[0, 0]
    cd, sd = cw.to(cuda)[:, :32], sw.to(cuda)[:, :32]
    assert cd.stride(0) == 35
    y = fused_rope(x.to(cuda), cd, sd).cpu()
    assert max_rel_err(y, ofo.rope(x.float(), cos, sin)) < 2e-2


def test_rope_strided_view_and_2d_cache(cuda):
    from hydra_amd.kernels import fused_rope

    g = _gen(4)
    base = torch.randn(2, 40, 6, 32, generator=g).to(torch.bfloat16)  # [B,S,H,D]
    x = base.transpose(1, 2)  # [B,H,S,D] view, non-contiguous
    cos, sin = ofo.rope_cache(32, 40)
    y = fused_rope(x.to(cuda), cos[0, 0].to(cuda), sin[0, 0].to(cuda)).cpu()
    assert max_rel_err(y, ofo.rope(x.float(), cos, sin)) < 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,hidden", [(16384, 2048), (1024, 1365), (3, 7), (1, 8)])
def test_swiglu_halves_of_gate_up(cuda, dtype, rows, hidden):
    from hydra_amd.kernels import fused_swiglu

    g = _gen(5)
    gu = (torch.randn(rows, 2 * hidden, generator=g) * 2).to(dtype)
    gate, up = gu.to(cuda).chunk(2, dim=-1)
    y = fused_swiglu(gate, up).cpu()
    gc, uc = gu.chunk(2, dim=-1)
    assert max_rel_err(y, ofo.swiglu(gc.float(), uc.float())) < TOL[dtype]
    assert max_rel_err(y, ofo.swiglu_fp32(gc, uc)) < (1e-6 if dtype == torch.float32 else 8e-3)


def test_swiglu_c2_shape(cuda):
    from hydra_amd.kernels import fused_swiglu

    g = _gen(6)
    gate = torch.randn(8, 2048, 2048, generator=g).to(torch.bfloat16)
    up = torch.randn(8, 2048, 2048, generator=g).to(torch.bfloat16)
    y = fused_swiglu(gate.to(cuda), up.to(cuda)).cpu()
    assert max_rel_err(y, ofo.swiglu(gate.float(), up.float())) < 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hd", [16, 64, 6, 128])
def test_qk_norm(cuda, dtype, hd):
    from hydra_amd.kernels import fused_qk_norm

    g = _gen(7)
    q = torch.randn(2, 8, 33, hd, generator=g).to(dtype)
    k = torch.randn(2, 2, 33, hd, generator=g).to(dtype)
    qo, ko = fused_qk_norm(q.to(cuda), k.to(cuda), 8.0, 0.5)
    rq, rk = ofo.qk_norm(q.float(), k.float(), 8.0, 0.5)
    assert max_rel_err(qo.cpu(), rq) < TOL[dtype]
    assert max_rel_err(ko.cpu(), rk) < TOL[dtype]


def test_cpu_tensor_raises():
    from hydra_amd.kernels import fused_rms_norm

    with pytest.raises(RuntimeError, match="GPU tensors only"):
        fused_rms_norm(torch.randn(2, 8), torch.ones(8))
