"""The CCGQA forward captured in a HIP graph (torch.cuda.graph) replays to
the eager result: several replays with eager work and synchronisations in
between, each compared bit for bit (the same kernels run on the same
inputs; every kernel on the path is deterministic), then a replay on new
input content against the eager forward of that content.  bench.py times
the config-3 step this way."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_ccgqa_forward_graph_replays_match_eager(cuda):
    from hydra_amd.attention import CCGQAAttention

    torch.manual_seed(3)
    m = CCGQAAttention(dim=1024, n_heads=4, n_kv_heads=1, compression_factor=4, max_seq_len=1024)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape) * 0.02)
        m.key_temperature.fill_(1.0)
    m = m.to(cuda, torch.bfloat16).eval()
    g = torch.Generator(device=cuda).manual_seed(4)
    x = torch.randn(2, 1024, 1024, device=cuda, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        m(x)
        want = m(x).clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            m(x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = m(x)
    for r in range(4):
        noise = torch.randn(4096, 4096, device=cuda, generator=g).sum()  # eager work between replays
        torch.cuda.synchronize()
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {r} differs from the eager forward"
        del noise
    x2 = torch.randn(x.shape, device=cuda, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        want2 = m(x2).clone()
    x.copy_(x2)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, want2)
    del graph


def test_hydra_model_forward_graph_replays_match_eager(cuda):
    """The config-5 model path (MoR blocks, MoD middle blocks, tied LM head)
    captured in a HIP graph: routing is capacity-based, so every shape is
    fixed and the forward has no host synchronisation.  Replays with eager
    work in between equal the eager logits bit for bit, and a replay on new
    token ids equals the eager forward of those ids.  bench.py times config
    5 this way."""
    from test_gpu_blocks import _model_from_checkpoint

    m, z, meta = _model_from_checkpoint(cuda, torch.bfloat16)
    g = torch.Generator(device=cuda).manual_seed(5)
    ids = torch.from_numpy(z["ids"]).to(cuda)
    with torch.no_grad():
        m(ids)
        want = m(ids).clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            m(ids)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = m(ids)
    for r in range(3):
        noise = torch.randn(4096, 4096, device=cuda, generator=g).sum()
        torch.cuda.synchronize()
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {r} differs from the eager forward"
        del noise
    ids2 = torch.randint(0, meta["vocab_size"], ids.shape, device=cuda, generator=g)
    with torch.no_grad():
        want2 = m(ids2).clone()
    ids.copy_(ids2)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, want2)
    del graph
