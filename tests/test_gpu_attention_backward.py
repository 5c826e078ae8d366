"""GPU parity of the CCGQA attention backward (hydra_attn_bwd) against the
oracle's restatement of the reference's split-K backward, on the same
bf16-rounded inputs (the oracle is pinned by autograd in
tests/test_oracle_pins.py).

The forward's log-sum-exp feeds the backward, as in the reference.
Tolerance: normwise max-rel-err < 2e-2 for bf16 (P and dS enter the MFMA
products in bf16, as in the reference's tl.dot), < 1e-5 for fp32 (VALU path,
fp32 throughout).  At the full config-3 shape the check is per batch against
the oracle plus two size-independent identities: sum_t dK[t] = 0 (each row of
dS sums to zero) and sum_t dV[t] = sum over the group's heads and rows of dO
(each row of P sums to one)."""
from __future__ import annotations

import pytest
import torch

from conftest import max_rel_err
from oracle import ccgqa as occ

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _inputs(B, Hq, Hkv, S, hd, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, S, hd, generator=g).to(dtype)
    k = torch.randn(B, Hkv, S, hd, generator=g).to(dtype)
    v = torch.randn(B, Hkv, S, hd, generator=g).to(dtype)
    go = torch.randn(B, Hq, S, hd, generator=g).to(dtype)
    return q, k, v, go


def _run(q, k, v, go, causal, cuda):
    from hydra_amd.attention.backends.ccgqa.ops import attention_backward, attention_forward

    qd, kd, vd, god = (t.to(cuda) for t in (q, k, v, go))
    out, lse = attention_forward(qd, kd, vd, causal=causal, want_lse=True)
    return attention_backward(qd, kd, vd, out, lse, god, causal=causal)


def _check(got, q, k, v, go, causal, tol):
    ref = occ.attention_backward(q, k, v, go, causal=causal)
    for name, a, r in zip(("dq", "dk", "dv"), got, ref):
        assert a.dtype == q.dtype and a.shape == r.shape
        err = max_rel_err(a.cpu(), r)
        assert err < tol, f"{name}: {err:.3g}"


# (B, Hq, Hkv, S, hd): GQA 4:1 (two key blocks x two head groups per
# workgroup), ragged S, MHA and odd G (four key blocks), G = 2, head_dim 32/128.
MFMA_CASES = [(2, 4, 1, 256, 64), (1, 8, 2, 300, 64), (2, 2, 2, 128, 128), (1, 3, 1, 200, 32),
              (1, 6, 3, 97, 64), (1, 4, 1, 1000, 128), (1, 1, 1, 33, 64)]


def test_attention_backward_many_heads(cuda):
    """B x Hq past 65535: the row-dot launch spreads (batch, head) over grid y
    and z."""
    q, k, v, go = _inputs(16400, 4, 1, 16, 32, torch.bfloat16, seed=7)
    _check(_run(q, k, v, go, True, cuda), q, k, v, go, True, TOL[torch.bfloat16])


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", MFMA_CASES)
def test_attention_backward_mfma(cuda, shape, causal):
    q, k, v, go = _inputs(*shape, torch.bfloat16, seed=sum(shape))
    _check(_run(q, k, v, go, causal, cuda), q, k, v, go, causal, TOL[torch.bfloat16])


# VALU path: fp32, and bf16 with head_dim outside {32, 64, 128} (config 0's
# debug shape has head_dim 16).
GENERIC_CASES = [(torch.float32, (1, 4, 2, 64, 16)), (torch.float32, (2, 2, 1, 37, 64)),
                 (torch.bfloat16, (2, 8, 2, 128, 16)), (torch.bfloat16, (1, 2, 1, 50, 48))]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype,shape", GENERIC_CASES)
def test_attention_backward_generic(cuda, dtype, shape, causal):
    q, k, v, go = _inputs(*shape, dtype, seed=sum(shape) + 1)
    _check(_run(q, k, v, go, causal, cuda), q, k, v, go, causal, TOL[dtype])


@pytest.mark.parametrize("use_fused_backward", [True, False])
def test_ccgqa_attention_fused_autograd(cuda, use_fused_backward):
    """The reference's public API (fused_attention.py:826-840) under autograd:
    loss.backward() fills q/k/v .grad through the HIP backward."""
    from hydra_amd.attention.backends.ccgqa.kernels import ccgqa_attention_fused

    q, k, v, go = _inputs(2, 4, 1, 192, 64, torch.bfloat16, seed=3)
    qd, kd, vd = (t.to(cuda).requires_grad_() for t in (q, k, v))
    out = ccgqa_attention_fused(qd, kd, vd, is_causal=True, use_fused_backward=use_fused_backward)
    out.backward(go.to(cuda))
    _check((qd.grad, kd.grad, vd.grad), q, k, v, go, True, TOL[torch.bfloat16])


def test_attention_backward_strided_and_deterministic(cuda):
    """q/k/v as [B,S,H,D] buffers seen transposed, grad_out non-contiguous;
    two calls give bit-identical gradients (no atomics)."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_backward, attention_forward

    q, k, v, go = _inputs(2, 4, 2, 160, 64, torch.bfloat16, seed=4)
    qd, kd, vd = (t.transpose(1, 2).contiguous().to(cuda).transpose(1, 2) for t in (q, k, v))
    god = go.transpose(1, 2).contiguous().to(cuda).transpose(1, 2)
    out, lse = attention_forward(qd, kd, vd, causal=True, want_lse=True)
    first = attention_backward(qd, kd, vd, out, lse, god, causal=True)
    second = attention_backward(qd, kd, vd, out, lse, god, causal=True)
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    _check(first, q, k, v, go, True, TOL[torch.bfloat16])


def test_attention_backward_config3_shape(cuda):
    """Config 3's attention (B 4, 4 query heads, 1 KV head, hd 64, S 4096,
    causal): batches 0 and 3 against the oracle, all four through the
    row-sum identities."""
    B, Hq, Hkv, S, hd = 4, 4, 1, 4096, 64
    q, k, v, go = _inputs(B, Hq, Hkv, S, hd, torch.bfloat16, seed=7)
    dq, dk, dv = _run(q, k, v, go, True, cuda)
    for b in (0, 3):
        _check((dq[b:b + 1], dk[b:b + 1], dv[b:b + 1]), q[b:b + 1], k[b:b + 1], v[b:b + 1],
               go[b:b + 1], True, TOL[torch.bfloat16])
    dk64, dv64 = dk.double().cpu(), dv.double().cpu()
    assert (dk64.sum(2).abs() / dk64.abs().sum(2)).max() < 1e-2
    want_v = go.double().view(B, Hkv, Hq // Hkv, S, hd).sum((2, 3))
    assert max_rel_err(dv64.sum(2), want_v) < 1e-2


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 8, 2, 300, 64), (1, 3, 1, 200, 32), (2, 2, 2, 130, 128)])
def test_attention_backward_query_chunks(cuda, monkeypatch, shape, causal):
    """dK/dV with each key group's query range cut into chunks of 3 tiles
    (fp32 partials summed in chunk order by the reduce launch), against the
    oracle; deterministic across calls."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_backward, attention_forward

    monkeypatch.setenv("HYDRA_ATTN_BWD_CHUNK", "3")
    q, k, v, go = _inputs(*shape, torch.bfloat16, seed=sum(shape) + 5)
    qd, kd, vd, god = (t.to(cuda) for t in (q, k, v, go))
    out, lse = attention_forward(qd, kd, vd, causal=causal, want_lse=True)
    first = attention_backward(qd, kd, vd, out, lse, god, causal=causal)
    second = attention_backward(qd, kd, vd, out, lse, god, causal=causal)
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    _check(first, q, k, v, go, causal, TOL[torch.bfloat16])


def test_attention_backward_two_streams(cuda):
    """Two backward calls queued on two user streams at once (both fork
    their dQ launch onto the library's one side stream per device): each
    equals the same call on the default stream, bit for bit."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_backward, attention_forward

    calls = []
    for seed in (21, 22):
        q, k, v, go = (t.to(cuda) for t in _inputs(2, 4, 1, 768, 64, torch.bfloat16, seed=seed))
        out, lse = attention_forward(q, k, v, causal=True, want_lse=True)
        calls.append((q, k, v, out, lse, go))
    want = [attention_backward(*c[:5], c[5], causal=True) for c in calls]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    got = []
    for st, c in zip(streams, calls):
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            got.append(attention_backward(*c[:5], c[5], causal=True))
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        for a, b in zip(g, w):
            assert torch.equal(a, b)


_CAPTURE_FIRST = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from hydra_amd.attention.backends.ccgqa.ops import attention_backward, attention_forward
g = torch.Generator().manual_seed(31)
q, k, v, go = (torch.randn(*sh, generator=g).to(torch.bfloat16).cuda()
               for sh in ((2, 4, 512, 64), (2, 1, 512, 64), (2, 1, 512, 64), (2, 4, 512, 64)))
out, lse = attention_forward(q, k, v, causal=True, want_lse=True)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(side):
    with torch.cuda.graph(graph):  # the process's first backward call
        got = attention_backward(q, k, v, out, lse, go, causal=True)
torch.cuda.current_stream().wait_stream(side)
torch.cuda.synchronize()
want = attention_backward(q, k, v, out, lse, go, causal=True)
for _ in range(3):
    for t in got:
        t.zero_()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(got, want))
print("capture-first ok")
"""


def test_attention_backward_captured_as_first_call(cuda):
    """A process whose first backward call is inside a graph capture (the
    library creates its side stream only outside one, so that call runs on
    the caller's stream alone): three replays equal the eager gradients."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    res = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST, root], capture_output=True, text=True,
                         timeout=180)
    assert res.returncode == 0 and "capture-first ok" in res.stdout, res.stdout[-2000:] + res.stderr[-2000:]


def test_attention_backward_in_hip_graph(cuda):
    """After one eager call (which sizes the library workspace), the backward
    captures into a HIP graph; three replays, with eager work and
    synchronisations between them, each equal the eager gradients bit for
    bit (no memset nodes: every output element is written by a kernel)."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_backward, attention_forward

    q, k, v, go = (t.to(cuda) for t in _inputs(2, 4, 1, 1024, 64, torch.bfloat16, seed=9))
    out, lse = attention_forward(q, k, v, causal=True, want_lse=True)
    want = attention_backward(q, k, v, out, lse, go, causal=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        attention_backward(q, k, v, out, lse, go, causal=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = attention_backward(q, k, v, out, lse, go, causal=True)
    for _ in range(3):
        for t in got:
            t.zero_()
        attention_backward(q, k, v, out, lse, go * 2, causal=True)  # eager work in between
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b)


MASK_CASES = [
    # B, Hq, Hkv, S, hd, dtype
    (2, 4, 2, 70, 32, torch.float32),
    (2, 4, 1, 96, 64, torch.bfloat16),
    (1, 6, 3, 40, 16, torch.float32),
]


@pytest.mark.parametrize("mode", ["key_padding", "reference"])
@pytest.mark.parametrize("case", MASK_CASES, ids=[str(c[:5]) for c in MASK_CASES])
def test_attention_backward_key_mask(cuda, case, mode):
    """hydra_attn_bwd with the forward's key mask: both mask modes against
    fp64 autograd through the oracle's masked forward (key padding: the
    explicit masked softmax attention_key_padding; reference: the SDPA call
    with the reference's combined attn_mask, attention.py:268-299).  Every
    row sees at least one key (key 0 kept; in the reference mode a padded
    key is visible to every row)."""
    from hydra_amd.attention.backends.ccgqa.ops import (MASK_KEY_PADDING, MASK_REFERENCE_SDPA,
                                                        attention_backward, attention_forward)

    B, Hq, Hkv, S, hd, dtype = case
    q, k, v, go = _inputs(B, Hq, Hkv, S, hd, dtype, seed=S + hd)
    g = torch.Generator().manual_seed(S)
    mask = (torch.rand(B, S, generator=g) > 0.3).long()
    mask[:, 0] = 1
    mask[:, S // 2] = 0
    mm = MASK_KEY_PADDING if mode == "key_padding" else MASK_REFERENCE_SDPA
    dev = lambda t: t.to(cuda)
    out, lse = attention_forward(dev(q), dev(k), dev(v), causal=True, key_mask=dev(mask), mask_mode=mm,
                                 want_lse=True)
    got = attention_backward(dev(q), dev(k), dev(v), out, lse, dev(go), causal=True, key_mask=dev(mask),
                             mask_mode=mm)
    q64, k64, v64 = (t.detach().double().requires_grad_(True) for t in (q, k, v))
    if mode == "key_padding":
        ref_out = occ.attention_key_padding(q64, k64, v64, causal=True, mask=mask)
    else:
        ref_out = occ.attention(q64, k64, v64, causal=True, mask=mask)
    assert max_rel_err(out.cpu(), ref_out.detach()) < TOL[dtype]
    ref_out.backward(go.double())
    for name, a, r in zip(("dq", "dk", "dv"), got, (q64.grad, k64.grad, v64.grad)):
        err = max_rel_err(a.cpu(), r)
        assert err < (1e-4 if dtype == torch.float32 else 5e-2), f"{name}: {err:.3g}"
