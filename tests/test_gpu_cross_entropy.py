"""GPU parity of the chunked LM-head cross-entropy (hydra_ce_rows plus the
GEMMs around it) against the oracle's fp64 restatement of
ChunkedCrossEntropyFunction (pinned by autograd of F.cross_entropy in
tests/test_oracle_pins.py): the loss and both gradients.  Tolerance: fp32
1e-5, bf16 2e-2 (max-rel-err; the forward's logits are bf16 GEMM outputs, as
in the reference)."""
from __future__ import annotations

import pytest
import torch

from conftest import max_rel_err
from oracle import fused_ops as ofo

pytestmark = pytest.mark.gpu


def _case(B, S, D, V, dtype, seed, ignore_frac=0.1):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(B, S, D, generator=g).to(dtype)
    w = (torch.randn(V, D, generator=g) * 0.05).to(dtype)
    t = torch.randint(0, V, (B, S), generator=g)
    t[torch.rand(B, S, generator=g) < ignore_frac] = -100
    return h, w, t


@pytest.mark.parametrize("dtype,shape,chunk", [
    (torch.float32, (2, 300, 64, 1000), 128),    # ragged last chunk
    (torch.float32, (1, 50, 32, 1001), 4096),    # one chunk, V not a multiple of 8
    (torch.bfloat16, (2, 256, 128, 32000), 192),  # LM-head vocab
])
def test_chunked_cross_entropy(cuda, dtype, shape, chunk):
    from hydra_amd.kernels import fused_chunked_cross_entropy

    h, w, t = _case(*shape, dtype, seed=sum(shape))
    hd, wd = h.to(cuda).requires_grad_(), w.to(cuda).requires_grad_()
    loss = fused_chunked_cross_entropy(hd, wd, t.to(cuda), chunk_size=chunk)
    loss.backward(torch.tensor(0.5, device=cuda, dtype=dtype))
    ref, gh, gw = ofo.chunked_cross_entropy(h, w, t, grad_output=0.5)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert loss.dtype == dtype
    assert abs(loss.item() - ref.item()) / abs(ref.item()) < tol
    assert max_rel_err(hd.grad.cpu(), gh) < tol
    assert max_rel_err(wd.grad.cpu(), gw) < tol


def test_chunked_cross_entropy_edge_targets(cuda):
    """All targets ignored: loss 0, zero gradients.  Out-of-range targets are
    clamped into [0, V) (fused_ops.py:1407-1422)."""
    from hydra_amd.kernels import chunked_cross_entropy

    h, w, t = _case(1, 40, 32, 100, torch.float32, seed=2)
    hd, wd = h.to(cuda).requires_grad_(), w.to(cuda).requires_grad_()
    loss = chunked_cross_entropy(hd, wd, torch.full_like(t, -100).to(cuda), chunk_size=16)
    loss.backward()
    assert loss.item() == 0 and hd.grad.abs().max() == 0 and wd.grad.abs().max() == 0
    t[0, 3], t[0, 9] = 150, -5
    hd.grad = wd.grad = None
    loss = chunked_cross_entropy(hd, wd, t.to(cuda), chunk_size=16)
    loss.backward()
    ref, gh, gw = ofo.chunked_cross_entropy(h, w, t)
    assert abs(loss.item() - ref.item()) / abs(ref.item()) < 1e-5
    assert max_rel_err(hd.grad.cpu(), gh) < 1e-5 and max_rel_err(wd.grad.cpu(), gw) < 1e-5


@pytest.mark.parametrize("oob", [False, True])
def test_token_losses_from_hidden(cuda, oob):
    """compute_token_losses_from_hidden (loop.py:28-89) against the oracle,
    fp32 throughout (1e-5), token chunks with a ragged tail."""
    from hydra_amd.training import compute_token_losses_from_hidden

    h, w, t = _case(2, 150, 64, 3000, torch.bfloat16, seed=21)
    if oob:
        t[1, 7] = 3005
    got = compute_token_losses_from_hidden(h.to(cuda), w.to(cuda), t.to(cuda), token_chunk_size=128)
    ref = ofo.token_losses_from_hidden(h.float(), w.float(), t)
    assert got.dtype == torch.float32 and got.shape == (2, 150)
    assert max_rel_err(got.cpu(), ref) < 1e-5
    assert (got.cpu()[ref == 0] == 0).all()


@pytest.mark.parametrize("V", [1000, 1001, 32000])
@pytest.mark.parametrize("with_grad", [False, True])
def test_ce_rows_masked_logits(cuda, V, with_grad):
    """hydra_ce_rows on logits holding -inf (masked vocabulary entries): whole
    16-byte chunks and single entries.  Loss and gradient must be those of
    F.cross_entropy in fp64 (finite; masked entries get zero gradient)."""
    from hydra_amd import _lib

    rows = 6
    g = torch.Generator().manual_seed(V)
    x = torch.randn(rows, V, generator=g)
    x[0, :64] = -float("inf")          # leading chunks fully masked
    x[1, 8:16] = -float("inf")         # one 16-byte chunk (fp32: two)
    x[2, torch.randperm(V, generator=g)[: V // 3]] = -float("inf")
    x[3, V - 5:] = -float("inf")       # ragged tail
    t = torch.randint(0, V, (rows,), generator=g)
    for r in range(4):
        while torch.isinf(x[r, t[r]]):
            t[r] = (t[r] + 1) % V
    t[5] = -100
    xd, td = x.to(cuda), t.to(cuda)
    loss = torch.empty(rows, device=cuda)
    grad = torch.empty_like(xd) if with_grad else None
    scale = torch.full((1,), 0.25, device=cuda)
    _lib.call("hydra_ce_rows", xd.data_ptr(), rows, V, V, td.data_ptr(), -100, loss.data_ptr(), None,
              grad.data_ptr() if with_grad else None, V, scale.data_ptr() if with_grad else None,
              _lib.dtype_code(xd), _lib.stream(xd))
    x64 = x.double()
    ref = torch.nn.functional.cross_entropy(x64, t, ignore_index=-100, reduction="none")
    assert torch.isfinite(loss.cpu()).all()
    assert max_rel_err(loss.cpu(), ref) < 1e-5
    if with_grad:
        p = torch.softmax(x64, -1)
        gr = p.clone()
        valid = t != -100
        gr[valid, t[valid]] -= 1
        gr[~valid] = 0
        gr *= 0.25
        gc = grad.cpu()
        assert torch.isfinite(gc).all()
        assert max_rel_err(gc, gr) < 1e-5
        assert (gc[torch.isinf(x)] == 0).all()
