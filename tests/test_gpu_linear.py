"""hydra_linear_fwd (the CCGQA output projection, attention.py:329-331)
against an fp32 reference product, through the C ABI and the module."""
import pytest
import torch
import torch.nn.functional as F

from conftest import max_rel_err

pytestmark = pytest.mark.gpu

CASES = [
    # M, N, K, x row stride (None: contiguous)
    (16384, 1024, 256, None),  # config 3's o_proj: 4 x 4096 tokens, latent 256 -> dim 1024
    (1000, 576, 256, None),    # ragged rows; a second workgroup with one active wave
    (300, 64, 128, 320),       # rows read from a wider buffer
    (77, 128, 64, None),
    (1, 512, 256, None),
]


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_linear_matches_fp32_product(cuda, case):
    from hydra_amd import _lib

    M, N, K, xrs = case
    g = torch.Generator().manual_seed(M + N + K)
    base = torch.randn(M, xrs or K, generator=g).to(torch.bfloat16)
    x = base[:, :K]
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    xd, wd = base.to(cuda)[:, :K], w.to(cuda)
    from hydra_amd.attention.backends.ccgqa.ops import pack_linear_weight

    y = torch.full((M, N), float("nan"), device=cuda, dtype=torch.bfloat16)
    _lib.call("hydra_linear_fwd", xd.data_ptr(), xd.stride(0), wd.data_ptr(), wd.stride(0), y.data_ptr(), N,
              M, N, K, 0, _lib.BF16, _lib.stream(xd))
    # the fragment-ordered weight gives the same bits
    yt = torch.full((M, N), float("nan"), device=cuda, dtype=torch.bfloat16)
    wt = pack_linear_weight(wd)
    _lib.call("hydra_linear_fwd", xd.data_ptr(), xd.stride(0), wt.data_ptr(), K, yt.data_ptr(), N,
              M, N, K, _lib.LINEAR_W_TILED, _lib.BF16, _lib.stream(xd))
    assert torch.equal(y, yt)
    ref = x.float() @ w.float().t()
    got = y.float().cpu()
    assert not torch.isnan(got).any()
    assert max_rel_err(got, ref) < 1e-2
    # the library GEMM on the same inputs (fp32 accumulation, one rounding):
    # at most a few bf16 ulps apart
    lib = F.linear(xd, wd).float().cpu()
    assert (got - lib).abs().max().item() <= 4 * 2 ** -8 * ref.abs().max().item()


def test_linear_unsupported_width_falls_back(cuda):
    from hydra_amd import _lib
    from hydra_amd.attention.backends.ccgqa.ops import output_projection

    x = torch.randn(64, 96, device=cuda).to(torch.bfloat16)
    w = torch.randn(128, 96, device=cuda).to(torch.bfloat16)
    y = torch.empty(64, 128, device=cuda, dtype=torch.bfloat16)
    rc = _lib.call_status("hydra_linear_fwd", x.data_ptr(), 96, w.data_ptr(), 96, y.data_ptr(), 128, 64, 128, 96,
                          0, _lib.BF16, _lib.stream(x))
    assert rc == _lib.ERR_UNSUPPORTED
    with torch.no_grad():
        assert torch.equal(output_projection(x, w), F.linear(x, w))


def test_output_projection_module_shape(cuda):
    """output_projection on a [B, S, L] activation (the module's call) equals
    the kernel on the flattened rows, and keeps F.linear under autograd."""
    from hydra_amd.attention.backends.ccgqa.ops import output_projection

    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 96, 256, generator=g).to(cuda, torch.bfloat16)
    w = (torch.randn(1024, 256, generator=g) * 0.05).to(cuda, torch.bfloat16)
    with torch.no_grad():
        y = output_projection(x, w)
    assert y.shape == (2, 96, 1024)
    ref = x.float().cpu() @ w.float().cpu().t()
    assert max_rel_err(y.float().cpu(), ref) < 1e-2
    wg = w.clone().requires_grad_(True)
    y2 = output_projection(x, wg)
    assert y2.grad_fn is not None
    y2.float().sum().backward()
    assert wg.grad is not None and wg.grad.shape == w.shape
