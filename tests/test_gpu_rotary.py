"""GPU tests of the RotaryEmbedding module (hydra/layers/common.py:242-338):
its fp32 cos/sin cache, the rotation it applies through fused_rope
(hydra_rope_fwd), cache extension past max_seq_len, and scaling_factor.

The cache is pinned by properties that a wrong index, sign or frequency
fails: cos^2 + sin^2 = 1, the angle of position p and pair i equals
p * base^(-2i/hd) / scaling (computed here in fp64), and the rotation
preserves every pair's norm and makes q.k depend only on the position
difference.  The rotation itself is checked against the oracle's restated
_rope_pytorch (fused_ops.py:300-306)."""
from __future__ import annotations

import math

import pytest
import torch

from conftest import max_rel_err
from oracle import fused_ops as ofo

pytestmark = pytest.mark.gpu


def test_rotary_cache_closed_form(cuda):
    from hydra_amd.layers import RotaryEmbedding

    hd, S, base = 64, 512, 10000.0
    rot = RotaryEmbedding(hd, max_seq_len=S, base=base)
    cos, sin = rot.get_cos_sin(S)
    assert cos.shape == (1, 1, S, hd // 2) and cos.dtype == torch.float32
    assert (cos.double() ** 2 + sin.double() ** 2 - 1).abs().max() < 1e-6
    pos = torch.arange(S, dtype=torch.float64)[:, None]
    i = torch.arange(hd // 2, dtype=torch.float64)[None]
    ang = pos * base ** (-2 * i / hd)
    # fp32 angles (product of fp32 inverse frequency and position) round to
    # within |ang| * 2^-23 of the fp64 angle
    tol = 2e-7 * ang.abs().max().item() + 1e-6
    assert (cos[0, 0].double() - ang.cos()).abs().max() < tol
    assert (sin[0, 0].double() - ang.sin()).abs().max() < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 4, 300, 64), (1, 8, 129, 16), (3, 2, 64, 128)])
def test_rotary_forward_matches_oracle(cuda, dtype, shape):
    from hydra_amd.layers import RotaryEmbedding

    B, H, S, hd = shape
    g = torch.Generator().manual_seed(S + hd)
    x = torch.randn(*shape, generator=g).to(dtype)
    rot = RotaryEmbedding(hd, max_seq_len=512).to(cuda)
    got = rot(x.to(cuda)).cpu()
    assert got.dtype == dtype
    cos, sin = rot.get_cos_sin(S)
    want = ofo.rope(x.float(), cos.cpu(), sin.cpu())
    assert max_rel_err(got, want) < (1e-5 if dtype == torch.float32 else 2e-2)
    # norm of every (2i, 2i+1) pair preserved
    pn = lambda t: t.double().view(B, H, S, hd // 2, 2).norm(dim=-1)
    assert (pn(got) - pn(x)).abs().max() < (1e-5 if dtype == torch.float32 else 2e-2)


def test_rotary_relative_position(cuda):
    """<rope(q) at m, rope(k) at n> depends on m - n only."""
    from hydra_amd.layers import RotaryEmbedding

    hd, S = 32, 200
    g = torch.Generator().manual_seed(1)
    q1, k1 = torch.randn(hd, generator=g), torch.randn(hd, generator=g)
    q = q1.expand(1, 1, S, hd).contiguous()
    k = k1.expand(1, 1, S, hd).contiguous()
    rot = RotaryEmbedding(hd, max_seq_len=S).to(cuda)
    rq, rk = rot(q.to(cuda)).cpu().double()[0, 0], rot(k.to(cuda)).cpu().double()[0, 0]
    for d in (0, 3, 17):
        dots = (rq[d:] * rk[: S - d]).sum(-1)
        assert (dots - dots[0]).abs().max() < 1e-3 * (q1.norm() * k1.norm()).item()
    # position 0 is the identity
    assert torch.equal(rq[0].float(), q1)


def test_rotary_extends_cache_on_device(cuda):
    """A sequence past max_seq_len rebuilds the cache (common.py:287-295) on
    the input's device, and the result equals a module built that long."""
    from hydra_amd.layers import RotaryEmbedding

    hd = 64
    x = torch.randn(1, 2, 100, hd, generator=torch.Generator().manual_seed(2)).to(cuda)
    short = RotaryEmbedding(hd, max_seq_len=32).to(cuda)
    long = RotaryEmbedding(hd, max_seq_len=100).to(cuda)
    got = short(x)
    assert short.max_seq_len == 100 and short.cos_cached.device == x.device
    assert torch.equal(got, long(x))


def test_rotary_scaling_factor(cuda):
    """scaling_factor s divides every frequency: position 2p under s = 2 has
    the angles of position p under s = 1 (both products exact in fp32)."""
    from hydra_amd.layers import RotaryEmbedding

    hd, S = 64, 256
    x = torch.randn(1, 1, S, hd, generator=torch.Generator().manual_seed(3)).to(cuda)
    r1 = RotaryEmbedding(hd, max_seq_len=S)
    r2 = RotaryEmbedding(hd, max_seq_len=2 * S, scaling_factor=2.0)
    c1, s1 = r1.get_cos_sin(S)
    c2, s2 = r2.get_cos_sin(2 * S)
    assert torch.equal(c2[:, :, ::2], c1) and torch.equal(s2[:, :, ::2], s1)
    assert not math.isclose(c2[0, 0, 1, 0].item(), c1[0, 0, 1, 0].item())
