"""Benchmark of the HYDRA hot path on one MI355X.

Headline (the JSON `value`): CCGQA attention forward tokens/s at config 3 --
dim 1024, 4x compression to latent 256, 4 query heads / 1 KV head (hd 64),
causal conv k=3, QK-mean, QK L2-norm with temperature 1.0, B4 x S4096, bf16,
random-init N(0, 0.02) weights, N(0,1) activations (seed 0).  A step is one
full module forward: qkv GEMM -> fused prep kernel -> attention kernel ->
o_proj GEMM, inputs resident in HBM (16 rotating input sets).  The K timed
steps are one HIP graph replay between synchronisations, so the graph's
launch latency (~0.1 ms for K = 100) is inside the timed region, spread
over the K steps; the eager Python-launched time is reported beside it.

Also reported on the same line:
  roofline      the attention op (dominant: the attention kernel and, when
                the stream-K schedule splits items, its merge kernel),
                algorithmic FLOPs / its average duration from HIP events
                recorded on the launch stream around a graph of
                back-to-back calls;
  stages        per-stage average durations of the eager step;
  fused_ops     config 2 RMSNorm / RoPE / SwiGLU in HBM GB/s and % of peak
                (buffers rotated over > 512 MB so the 256 MB MALL cannot
                serve repeats), each beside the same-device time of a plain
                non-temporal copy of its bytes (copy_ms, pct_of_copy);
  mod           config 4 top-k / gather / residual scatter (with the same
                copy figures);
  c1_block      config 1: embedding + HydraBlock (CCGQA dim 512, 8/2 heads
                of 16, SwiGLU hidden 1365) forward in fp32, B2 x S512,
                tokens/s (a HIP graph of the steps), with the oracle's CPU
                figure for the same workload;
  c5_model      config 5: HydraModel forward in bf16 at the 1B shape (dim
                1792, 20 MoR blocks x 4 recursions, MoD 0.75 in the middle
                blocks, vocab 32000), B4 x S4096, tokens/s;
  cpu_baseline  the oracle (the reference's PyTorch CPU path restated) on a
                bounded sample of the same workload, on this host's cores;
                cpu_baselines adds configs 1, 2 and 4 the same way.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                      [--only-c3] [--only-attn-bwd] [--no-c5]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch
import torch.nn.functional as F

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "CCGQA block fwd tokens/s + fused-op HBM GB/s (% peak), 1xMI355X"


def _events(n):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


# ----------------------------------------------------------------- config 3
class C3Step:
    """One CCGQA attention forward at config 3, stage by stage."""

    def __init__(self, dev, B=4, S=4096, dim=1024, n_heads=4, n_kv_heads=1, comp=4, seed=0,
                 temperature=1.0):
        from hydra_amd.attention import CCGQAAttention

        g = torch.Generator().manual_seed(seed)
        self.B, self.S, self.dim = B, S, dim
        m = CCGQAAttention(dim=dim, n_heads=n_heads, n_kv_heads=n_kv_heads,
                           compression_factor=comp, max_seq_len=S)
        with torch.no_grad():
            x = torch.randn(B, S, dim, generator=g)
            for name, p in m.named_parameters():
                if name == "key_temperature":
                    p.fill_(temperature)
                else:
                    p.copy_(torch.randn(p.shape, generator=g) * 0.02)
        self.m = m.to(dev, torch.bfloat16).eval()
        self.x = x.to(dev, torch.bfloat16)
        from hydra_amd.attention.backends.ccgqa.ops import prep_flags

        from hydra_amd._lib import CCGQA_V_TRANSPOSED, CCGQA_W_TILED
        from hydra_amd.attention.backends.ccgqa.ops import tiled_weights_ok

        self.flags = prep_flags(True, True, True, True, True) | CCGQA_V_TRANSPOSED
        mm = self.m
        tiled = tiled_weights_ok(n_heads, n_kv_heads, mm.head_dim, torch.bfloat16)
        if tiled:
            self.flags |= CCGQA_W_TILED
        self.convw = mm._packed_conv_weights((mm.q_conv.conv1.weight, mm.q_conv.conv2.weight,
                                              mm.k_conv.conv1.weight, mm.k_conv.conv2.weight),
                                             torch.bfloat16, tiled)
        self.cos = mm.cos_cached[0, 0, :S].float().contiguous()
        self.sin = mm.sin_cached[0, 0, :S].float().contiguous()
        self.out = torch.empty(B, S, mm.latent_dim, dtype=torch.bfloat16, device=dev)
        # |q.k| bound from QK-norm, taken by the kernel from the temperature
        self.temp = mm.key_temperature.detach()
        # o_proj weight in the output-projection kernel's fragment order
        self.w_o = mm._packed_o_proj()

    @torch.no_grad()
    def __call__(self, ev=None, x=None):
        from hydra_amd.attention.backends.ccgqa.ops import attention_forward, ccgqa_prep, output_projection

        m = self.m
        if ev:
            ev[0].record()
        qkv = F.linear(self.x if x is None else x, m.qkv_proj.weight)
        if ev:
            ev[1].record()
        q, k, v = ccgqa_prep(qkv, m.n_heads, m.n_kv_heads, m.head_dim, self.flags, *self.convw,
                             temperature=m.key_temperature, cos=self.cos, sin=self.sin,
                             packed=True)
        if ev:
            ev[2].record()
        o_view = self.out.view(self.B, self.S, m.n_heads, m.head_dim).transpose(1, 2)
        attention_forward(q, k, v, causal=True, scale=m.scale, out=o_view, bound_temperature=self.temp)
        if ev:
            ev[3].record()
        y = output_projection(self.out, m.o_proj.weight, self.w_o)
        if ev:
            ev[4].record()
        return y


def c3_flops(B=4, S=4096, dim=1024, Hq=4, Hkv=1, comp=4, ks=3):
    """Algorithmic FLOPs of one config-3 forward (multiply-add = 2).  The
    latent is dim/comp wide, split into Hq heads of hd = latent/Hq; K and V
    are Hkv*hd wide.  Each conv sequence is a grouped k=3 conv (hd inputs
    per output channel) followed by a dense k=3 conv; the attention core is
    causal QK^T + PV over S(S+1)/2 (query, key) pairs per head."""
    L = dim // comp
    hd = L // Hq
    K = Hkv * hd
    N = B * S
    f = {
        "qkv_proj": 2 * N * dim * (L + 2 * K),
        "q_conv": 2 * N * ks * (L * hd + L * L),
        "k_conv": 2 * N * ks * (K * hd + K * K),
        "core": 4 * B * Hq * hd * S * (S + 1) // 2,
        "o_proj": 2 * N * L * dim,
    }
    f["total"] = sum(f.values())
    return f


N_X_SETS = 16  # rotating input sets: 16 x 32 MiB, more than the 256 MiB MALL holds


def time_prep_and_attention(step, iters):
    """Average durations (ms) of the prep kernel and of the attention op of
    a C3Step's module, each timed alone as back-to-back calls."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward, ccgqa_prep

    m = step.m
    with torch.no_grad():
        qkv = F.linear(step.x, m.qkv_proj.weight)
        prep = lambda: ccgqa_prep(qkv, m.n_heads, m.n_kv_heads, m.head_dim, step.flags, *step.convw,
                                  temperature=m.key_temperature, cos=step.cos, sin=step.sin,
                                  packed=True)
        q, k, v = prep()
        prep_ms = _time_rotating(prep, [()], iters)
        o_view = step.out.view(step.B, step.S, m.n_heads, m.head_dim).transpose(1, 2)
        attn_ms = _time_rotating(lambda: attention_forward(q, k, v, causal=True, scale=m.scale, out=o_view,
                                                           bound_temperature=step.temp),
                                 [()], iters)
    return prep_ms, attn_ms


def shader_clock_mhz(dev, iters=200, reps=5):
    """The shader clock under a synthetic matrix-core load
    (hydra_clock_probe: two 8-wave workgroups per CU issuing bf16 MFMAs and
    v_exp_f32), median over `reps` back-to-back probes: sum of s_memtime
    ticks over sum of s_memrealtime ticks, times the wall clock's rate.
    Returns (MHz, wall-clock rate in kHz)."""
    import ctypes

    from hydra_amd import _lib

    nwg = 2 * torch.cuda.get_device_properties(dev).multi_processor_count
    stamps = torch.zeros(nwg * 5, dtype=torch.int64, device=dev)
    khz = ctypes.c_int64(0)
    vals = []
    for _ in range(reps):
        _lib.call("hydra_clock_probe", stamps.data_ptr(), nwg, iters, ctypes.byref(khz), _lib.stream(stamps))
        st = stamps.view(nwg, 5).cpu()
        shader = (st[:, 1] - st[:, 0]).double().sum().item()
        wall = (st[:, 3] - st[:, 2]).double().sum().item()
        vals.append(shader / wall * khz.value / 1e3)
    vals.sort()
    return vals[len(vals) // 2], khz.value


def attention_clock(step, wall_khz, reps=5):
    """The shader clock the key-split attention kernel itself runs at: its
    workgroups stamp s_memtime and s_memrealtime at start and end
    (hydra_attn_clock_stamps), over `reps` back-to-back launches; returns
    (MHz = sum of shader ticks / sum of wall ticks x wall rate, mean
    first-start-to-last-end span of a launch in ms)."""
    from hydra_amd import _lib
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward, ccgqa_prep

    m = step.m
    cap = 1 << 16
    buf = torch.zeros(reps, cap * 4, dtype=torch.int64, device=step.x.device)
    with torch.no_grad():
        qkv = F.linear(step.x, m.qkv_proj.weight)
        q, k, v = ccgqa_prep(qkv, m.n_heads, m.n_kv_heads, m.head_dim, step.flags, *step.convw,
                             temperature=m.key_temperature, cos=step.cos, sin=step.sin, packed=True)
        o_view = step.out.view(step.B, step.S, m.n_heads, m.head_dim).transpose(1, 2)
        attention_forward(q, k, v, causal=True, scale=m.scale, out=o_view, bound_temperature=step.temp)
        try:
            for r in range(reps):
                _lib.call("hydra_attn_clock_stamps", buf[r].data_ptr(), cap)
                attention_forward(q, k, v, causal=True, scale=m.scale, out=o_view,
                                  bound_temperature=step.temp)
        finally:
            _lib.call("hydra_attn_clock_stamps", None, 0)
    torch.cuda.synchronize()
    st = buf.view(reps, cap, 4).cpu()
    used = st[0, :, 3] != 0
    st = st[:, used]
    shader = (st[..., 1] - st[..., 0]).double().sum().item()
    wall = (st[..., 3] - st[..., 2]).double().sum().item()
    span = ((st[..., 3].max(1).values - st[..., 2].min(1).values).double().mean().item()
            / wall_khz)
    return shader / wall * wall_khz / 1e3, span


def bench_c3(dev, steps, warmup):
    """The config-3 step timed two ways over rotating inputs (one x per step,
    N_X_SETS sets, so repeats are not served from the memory-side cache):

    - graph: the K steps captured into one HIP graph and replayed (after W
      eager warmup steps and one untimed replay) -- the GPU timeline of the
      steps without the host's Python/ctypes launch cost, one graph launch
      for all K.  This is the reported value.
    - eager: the same K steps launched from Python, with HIP events around
      each stage (the stage breakdown; host launch gaps included).

    The attention stage is also timed on its own as a graph of back-to-back
    calls (the roofline's avg_ms), which is what the kernel trace's average
    durations of its two kernels add up to."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_forward, ccgqa_prep

    step = C3Step(dev)
    g = torch.Generator(device=dev).manual_seed(1)
    xs = [step.x] + [torch.randn(step.x.shape, device=dev, generator=g).to(torch.bfloat16)
                     for _ in range(N_X_SETS - 1)]
    check = step()  # also warms the GEMM heuristics and sizes the attention workspace
    del check
    for i in range(warmup):
        step(x=xs[i % N_X_SETS])
    torch.cuda.synchronize()
    # eager, with per-stage events
    evs = [_events(5) for _ in range(steps)]
    t0, t1 = _events(2)
    torch.cuda.synchronize()
    t0.record()
    for i in range(steps):
        step(evs[i], x=xs[i % N_X_SETS])
    t1.record()
    torch.cuda.synchronize()
    eager_ms = t0.elapsed_time(t1) / steps
    names = ["qkv_gemm", "prep", "attention", "o_proj_gemm"]
    stages = {n: sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps for j, n in enumerate(names)}
    # graph: the K steps (input sets in turn) captured into one HIP graph,
    # replayed once untimed and once timed -- exactly K steps, one graph
    # launch for all of them
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(2):
            step(x=xs[i])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            step(x=xs[i % N_X_SETS])
    graph.replay()
    torch.cuda.synchronize()
    t0, t1 = _events(2)
    t0.record()
    graph.replay()
    t1.record()
    torch.cuda.synchronize()
    graph_ms = t0.elapsed_time(t1) / steps
    del graph
    # the attention op alone, back to back in a graph
    m = step.m
    with torch.no_grad():
        qkv = F.linear(step.x, m.qkv_proj.weight)
        q, k, v = ccgqa_prep(qkv, m.n_heads, m.n_kv_heads, m.head_dim, step.flags, *step.convw,
                             temperature=m.key_temperature, cos=step.cos, sin=step.sin, packed=True)
    o_view = step.out.view(step.B, step.S, m.n_heads, m.head_dim).transpose(1, 2)
    attn_ms = _time_rotating(lambda: attention_forward(q, k, v, causal=True, scale=m.scale, out=o_view,
                                                       bound_temperature=step.temp),
                             [()], 8 * max(1, steps // 2))
    return step, graph_ms, eager_ms, stages, attn_ms


# ----------------------------------------------------------------- config 2
def _time_rotating(fn, sets, iters, warmup=3):
    """Average GPU time per call of fn over rotating argument sets.

    The calls are captured once into a HIP graph (torch.cuda.graph) and the
    graph is replayed, so the figure is kernel time on the GPU timeline and
    not the Python/ctypes launch cost, which exceeds a ~10 us kernel.  The
    graph holds at least 96 calls, so the gap at each replay boundary is
    spread over as many calls (with 12 calls per graph a ~9 us kernel read
    ~0.3 us longer)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(warmup):
            fn(*sets[i % len(sets)])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    n_per = max(len(sets), 96)
    with torch.cuda.graph(graph):
        for i in range(n_per):
            fn(*sets[i % len(sets)])
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, iters // n_per)
    a, b = _events(2)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / (reps * n_per)
    del graph
    return ms


def bench_fused_ops(dev, iters=60):
    from hydra_amd.kernels import fused_rms_norm, fused_rope, fused_swiglu
    from oracle.fused_ops import rope_cache

    g = torch.Generator(device=dev).manual_seed(0)
    res = {}
    N, D, H = 8 * 2048, 768, 2048
    bf = torch.bfloat16
    # RMSNorm [8,2048,768]: 12 x (25 MB in + 25 MB out) rotating sets
    w = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(bf)
    sets = [(torch.randn(8, 2048, D, device=dev, generator=g).to(bf), w) for _ in range(12)]
    ms = _time_rotating(lambda x, w: fused_rms_norm(x, w, 1e-6), sets, iters)
    nbytes = 2 * N * D * 2 + 2 * D
    res["rms_norm"] = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6}
    del sets
    # RoPE [8,12,2048,64] with fp32 [2048,32] cos/sin
    cos, sin = rope_cache(64, 2048)
    cos, sin = cos[0, 0].to(dev), sin[0, 0].to(dev)
    sets = [(torch.randn(8, 12, 2048, 64, device=dev, generator=g).to(bf),) for _ in range(12)]
    ms = _time_rotating(lambda x: fused_rope(x, cos, sin), sets, iters)
    nbytes = 2 * 8 * 12 * 2048 * 64 * 2 + 2 * 2048 * 32 * 4
    res["rope"] = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6}
    del sets
    # SwiGLU: halves of gate_up [8,2048,4096] -> [8,2048,2048]; 4 rotating sets
    sets = []
    for _ in range(4):
        gu = torch.randn(8, 2048, 2 * H, device=dev, generator=g).to(bf)
        sets.append(tuple(gu.chunk(2, -1)))
    ms = _time_rotating(lambda a, b: fused_swiglu(a, b), sets, iters)
    nbytes = 3 * N * H * 2
    res["swiglu"] = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6}
    del sets
    res.update(_bench_fused_backward(dev, g, iters))
    for v in res.values():
        v["pct_peak"] = 100.0 * v["GBs"] / HBM_PEAK_GBS
    _annotate_copy_ceiling(dev, res, iters)
    return res


def _copy_ceiling_ms(dev, nbytes, iters):
    """Time of hydra_stream_copy moving nbytes in total (half read, half
    written) on this device, with rotating buffers (>= ~600 MB, past the
    L2 and the 256 MB Infinity Cache), graph-replayed like the kernels."""
    from hydra_amd import _lib

    half = (nbytes // 2 + 15) // 16 * 16
    nsets = max(4, -(-600_000_000 // (2 * half)))
    sets = [(torch.empty(half, dtype=torch.uint8, device=dev), torch.empty(half, dtype=torch.uint8, device=dev))
            for _ in range(nsets)]
    ms = _time_rotating(lambda a, b: _lib.call("hydra_stream_copy", a.data_ptr(), b.data_ptr(), half,
                                               _lib.stream(a)), sets, iters)
    del sets
    return ms


def _annotate_copy_ceiling(dev, res, iters):
    """Per HBM-bound kernel: the same-device copy time of its algorithmic
    bytes (half each way) and the kernel's rate as a percentage of that
    copy's -- the practical ceiling of a one-pass kernel, which varies from
    box to box (62-73% of 8 TB/s measured at ~50 MB)."""
    cache = {}
    for v in res.values():
        if "GBs" not in v:
            continue
        nb = v["bytes"]
        if nb not in cache:
            cache[nb] = _copy_ceiling_ms(dev, nb, iters)
        v["copy_ms"] = cache[nb]
        v["copy_pct_peak"] = 100.0 * nb / cache[nb] / 1e6 / HBM_PEAK_GBS
        v["pct_of_copy"] = 100.0 * cache[nb] / v["ms"]


def bench_attention_backward(dev, iters=20):
    """CCGQA attention backward (hydra_attn_bwd) at config 3's attention
    shape: B 4, 4 query heads, 1 KV head, hd 64, S 4096, causal, bf16.
    Algorithmic flops: the five causal products (S, dP, dV, dK, dQ),
    5 * 2 * B * Hq * S^2 / 2 * hd.  Timed with events around `iters` calls
    (each call: row-dot, dK/dV, chunk reduce and dQ launches)."""
    from hydra_amd.attention.backends.ccgqa.ops import attention_backward, attention_forward

    B, Hq, Hkv, S, hd = 4, 4, 1, 4096, 64
    g = torch.Generator(device=dev).manual_seed(3)
    q, do = (torch.randn(B, Hq, S, hd, device=dev, generator=g).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn(B, Hkv, S, hd, device=dev, generator=g).to(torch.bfloat16) for _ in range(2))
    out, lse = attention_forward(q, k, v, causal=True, want_lse=True)
    for _ in range(3):
        attention_backward(q, k, v, out, lse, do, causal=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        attention_backward(q, k, v, out, lse, do, causal=True)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    flops = 5 * 2 * B * Hq * S * S / 2 * hd
    tf = flops / (ms * 1e-3) / 1e12
    return {"shape": "B4 Hq4 Hkv1 S4096 hd64 causal bf16", "ms": ms, "flops": flops,
            "TFLOPs": tf, "frac_bf16_peak": tf / BF16_PEAK_TFLOPS}


def bench_cross_entropy(dev, iters=20):
    """hydra_ce_rows on one chunk of the LM-head loss: 4096 tokens x vocab
    32000.  Forward: bf16 logits -> per-row loss (algorithmic bytes: the
    logits read once).  Backward: fp32 logits rewritten in place with their
    gradient (read once + written once; the kernel's second read of a row
    mostly hits L2/MALL)."""
    from hydra_amd import _lib

    rows, V = 4096, 32000
    g = torch.Generator(device=dev).manual_seed(5)
    t = torch.randint(0, V, (rows,), device=dev, generator=g)
    loss = torch.empty(rows, device=dev)
    scale = torch.full((1,), 1.0 / rows, device=dev)
    res = {"shape": "4096 tokens x vocab 32000"}
    for name, dt, grad in (("forward_bf16", torch.bfloat16, False), ("backward_fp32", torch.float32, True)):
        sets = [torch.randn(rows, V, device=dev, generator=g).to(dt) for _ in range(2)]
        call = lambda x: _lib.call("hydra_ce_rows", x.data_ptr(), rows, V, V, t.data_ptr(), -100,
                                   loss.data_ptr(), None, x.data_ptr() if grad else None, V,
                                   scale.data_ptr() if grad else None, _lib.dtype_code(x), _lib.stream(x))
        ms = _time_rotating(call, [(x,) for x in sets], iters)
        nbytes = rows * V * sets[0].element_size() * (2 if grad else 1)
        res[name] = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6,
                     "pct_peak": nbytes / ms / 1e6 / 8000 * 100}
        del sets
    return res


def _bench_fused_backward(dev, g, iters):
    """The backward kernels at the config-2 shapes, called through the C ABI
    on preallocated buffers (algorithmic bytes: every input read once, every
    output written once)."""
    from hydra_amd import _lib
    from oracle.fused_ops import rope_cache

    res = {}
    bf = torch.bfloat16
    N, D, H = 8 * 2048, 768, 2048
    st = lambda t: _lib.stream(t)
    # RMSNorm backward [16384, 768]: x, grad_y -> grad_x, grad_w
    w = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(bf)
    gw = torch.empty(D, device=dev, dtype=bf)
    sets = [(torch.randn(N, D, device=dev, generator=g).to(bf), torch.randn(N, D, device=dev, generator=g).to(bf),
             torch.empty(N, D, device=dev, dtype=bf)) for _ in range(6)]
    need = _lib.query("hydra_rms_norm_bwd_workspace", N, D)
    ws = _lib.scratch(need, w)
    ms = _time_rotating(lambda x, gy, gx: _lib.call(
        "hydra_rms_norm_bwd", x.data_ptr(), w.data_ptr(), gy.data_ptr(), gx.data_ptr(), gw.data_ptr(),
        N, D, D, D, D, 1e-6, _lib.dtype_code(x), _lib.dtype_code(w), ws.data_ptr(), need, st(x)), sets, iters)
    nbytes = 3 * N * D * 2 + 2 * D * 2
    res["rms_norm_bwd"] = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6}
    del sets
    # RoPE backward [8,12,2048,64]
    cos, sin = rope_cache(64, 2048)
    cos, sin = cos[0, 0].to(dev), sin[0, 0].to(dev)
    shape = (8, 12, 2048, 64)
    strides = lambda t: _lib.strides(t)
    sets = [(torch.randn(*shape, device=dev, generator=g).to(bf), torch.empty(shape, device=dev, dtype=bf))
            for _ in range(6)]
    ms = _time_rotating(lambda gy, gx: _lib.call(
        "hydra_rope_bwd", gy.data_ptr(), cos.data_ptr(), sin.data_ptr(), gx.data_ptr(), 8, 12, 2048, 64,
        strides(gy), cos.stride(0), _lib.dtype_code(gy), _lib.dtype_code(cos), st(gy)), sets, iters)
    nbytes = 2 * 8 * 12 * 2048 * 64 * 2 + 2 * 2048 * 32 * 4
    res["rope_bwd"] = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6}
    del sets
    # SwiGLU backward: halves of gate_up [16384, 4096], grad_y [16384, 2048]
    # -> grad_gate_up [16384, 4096]
    sets = []
    for _ in range(2):
        gu = torch.randn(N, 2 * H, device=dev, generator=g).to(bf)
        gy = torch.randn(N, H, device=dev, generator=g).to(bf)
        sets.append((gu, gy, torch.empty(N, 2 * H, device=dev, dtype=bf)))
    ms = _time_rotating(lambda gu, gy, gg: _lib.call(
        "hydra_swiglu_bwd", gu.data_ptr(), gu[:, H:].data_ptr(), gy.data_ptr(), gg.data_ptr(),
        gg[:, H:].data_ptr(), N, H, 2 * H, 2 * H, H, 2 * H, 2 * H, _lib.dtype_code(gu), st(gu)), sets, iters)
    nbytes = 5 * N * H * 2
    res["swiglu_bwd"] = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6}
    del sets
    return res


# ----------------------------------------------------------------- config 4
def bench_mod(dev, iters=50):
    from hydra_amd.routing import gather_by_indices, mod_topk, weighted_residual_scatter
    from oracle.mod import make_tied_logits

    g = torch.Generator().manual_seed(0)
    B, L, D, k = 8, 4096, 1280, 3072
    scores = make_tied_logits(B, L, 0.05, g).to(dev)
    res = {}
    ms = _time_rotating(lambda s: mod_topk(s, k), [(scores,)], iters)
    res["topk"] = {"ms": ms, "bytes": B * L * 4 + 2 * B * k * 8, "us": ms * 1e3}
    _, idx, _ = mod_topk(scores, k)
    gd = torch.Generator(device=dev).manual_seed(1)
    xs = [torch.randn(B, L, D, device=dev, generator=gd).to(torch.bfloat16) for _ in range(4)]
    ys = [torch.randn(B, k, D, device=dev, generator=gd).to(torch.bfloat16) for _ in range(4)]
    ms = _time_rotating(lambda x: gather_by_indices(x, idx), [(x,) for x in xs], iters)
    nb = 2 * B * k * D * 2
    res["gather"] = {"ms": ms, "bytes": nb, "GBs": nb / ms / 1e6, "pct_peak": 100 * nb / ms / 1e6 / HBM_PEAK_GBS}
    ms = _time_rotating(lambda h, y: weighted_residual_scatter(h, y, idx), list(zip(xs, ys)), iters)
    nb = 3 * B * k * D * 2
    res["scatter"] = {"ms": ms, "bytes": nb, "GBs": nb / ms / 1e6, "pct_peak": 100 * nb / ms / 1e6 / HBM_PEAK_GBS}
    _annotate_copy_ceiling(dev, res, iters)
    return res


# ------------------------------------------------------------- CPU baseline
def host_cpu() -> dict:
    """This host's CPU as the baseline reports it: model name, family / model
    / stepping, physical and logical cores, the CPUs this process may run on, ISA extensions that
    matter for torch's CPU kernels, and the threads the baselines use.
    Threads: the CPUs this process may use, capped by OMP_NUM_THREADS when
    the environment sets it (a GPU box shares its host between GPUs) and by
    the physical core count (no SMT siblings)."""
    info = {"model": "unknown", "physical_cores": None, "logical_cores": os.cpu_count(),
            "usable_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None}
    flags, cores = set(), set()
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name" and info["model"] == "unknown":
                info["model"] = val
            elif key in ("cpu family", "model", "stepping"):
                name = {"cpu family": "cpu_family", "model": "cpu_model", "stepping": "stepping"}[key]
                info.setdefault(name, int(val) if val.isdigit() else val)
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
                cores.add((phys, core))
            elif key == "flags" and not flags:
                flags = set(val.split())
    except OSError:
        pass
    info["physical_cores"] = len(cores) or None
    info["isa"] = {f: f in flags for f in ("avx2", "avx512f", "avx512_bf16", "amx_bf16", "amx_tile")}
    # family 26 (0x1A) is AMD Zen 5 (EPYC 9005); a guest names only "AMD EPYC"
    info["virtualised"] = "hypervisor" in flags
    threads = info["usable_cpus"] or info["logical_cores"] or 1
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    if info["physical_cores"]:
        threads = min(threads, info["physical_cores"])
    info["threads"] = max(1, threads)
    info["torch"] = torch.__version__
    return info


def _median_time(fn, budget_s, min_runs=5, max_runs=200, warmup=2):
    for _ in range(warmup):
        fn()
    times = []
    start = time.perf_counter()
    while len(times) < min_runs or ((time.perf_counter() - start) < budget_s and len(times) < max_runs):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return sorted(times)[len(times) // 2], len(times), time.perf_counter() - start


def cpu_baseline(host: dict, budget_s=12.0):
    """The oracle (reference PyTorch CPU path restated) on the config 3
    workload (B=4 x S=4096, bf16): tokens/s on this host, median over repeats
    bounded by budget_s seconds."""
    from oracle import ccgqa as occ

    torch.set_num_threads(host["threads"])
    cfg = occ.CCGQAConfig(dim=1024, n_heads=4, n_kv_heads=1, compression_factor=4, max_seq_len=4096)
    g = torch.Generator().manual_seed(0)
    params = {k: v.to(torch.bfloat16) for k, v in occ.init_params(cfg, g, temperature=1.0).items()}
    B, S = 4, 4096
    x = torch.randn(B, S, 1024, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        med, n, el = _median_time(lambda: occ.forward(params, x, cfg), budget_s)
    return {"value": B * S / med, "unit": "tokens/s", "cores": host["threads"], "kind": "port",
            "sample": f"oracle CCGQA forward (attention.py:201-331 restated on torch CPU ops), "
                      f"full config 3 (B=4 x S=4096, bf16); median of {n} runs in {el:.1f} s",
            "host": host}


def cpu_baselines(host: dict, budget_s=6.0) -> dict:
    """Configs 1, 2 and 4 on the oracle (the reference's CPU ops) in their
    own dtypes, same host and threads as cpu_baseline."""
    import math

    from oracle import blocks as ob
    from oracle import ccgqa as occ
    from oracle import fused_ops as ofo
    from oracle import mod as omod

    torch.set_num_threads(host["threads"])
    res = {}
    g = torch.Generator().manual_seed(0)
    # config 1: embedding + HydraBlock, fp32, B2 x S512
    cfg = occ.CCGQAConfig(dim=512, n_heads=8, n_kv_heads=2, compression_factor=4, max_seq_len=512)
    p = {"attention." + k: v for k, v in occ.init_params(cfg, g, temperature=4.0).items()}
    p.update({"norm1.weight": torch.ones(512), "norm2.weight": torch.ones(512),
              "mlp.gate_up.weight": torch.randn(2 * 1365, 512, generator=g) * 0.02,
              "mlp.down.weight": torch.randn(512, 1365, generator=g) * 0.02,
              "tok_emb.weight": torch.randn(32000, 512, generator=g) * 0.02})
    ids = torch.randint(0, 32000, (2, 512), generator=g)
    with torch.no_grad():
        med, n, _ = _median_time(lambda: ob.c1_forward(p, ids, cfg), budget_s)
    res["c1_block"] = {"value": 1024 / med, "unit": "tokens/s", "dtype": "fp32",
                       "sample": f"full config 1 (B2 x S512), median of {n}"}
    # config 2: RMSNorm / RoPE / SwiGLU activation, bf16, full shapes
    bf = torch.bfloat16
    x = torch.randn(8, 2048, 768, generator=g).to(bf)
    w = (1 + 0.1 * torch.randn(768, generator=g)).to(bf)
    xr = torch.randn(8, 12, 2048, 64, generator=g).to(bf)
    cos, sin = ofo.rope_cache(64, 2048)
    gate = torch.randn(8, 2048, 2048, generator=g).to(bf)
    up = torch.randn(8, 2048, 2048, generator=g).to(bf)
    for name, fn, nbytes in (
            ("rms_norm", lambda: ob.rms_norm(x, w, 1e-6), 50_333_184),
            ("rope", lambda: ofo.rope(xr, cos, sin), 50_855_936),
            ("swiglu", lambda: F.silu(gate) * up, 201_326_592)):
        med, n, _ = _median_time(fn, budget_s / 3)
        res[name] = {"ms": med * 1e3, "GBs": nbytes / med / 1e9, "dtype": "bf16",
                     "sample": f"full config 2 shape, median of {n}"}
    # config 4: top-k (torch.topk + mask), gather, residual scatter, bf16 rows
    scores = omod.make_tied_logits(8, 4096, 0.05, g)
    xs = torch.randn(8, 4096, 1280, generator=g).to(bf)
    ys = torch.randn(8, 3072, 1280, generator=g).to(bf)
    idx = torch.topk(scores, 3072, dim=-1).indices.sort(dim=1).values
    ie = idx.unsqueeze(-1).expand(-1, -1, 1280)

    def topk():
        _, ti = torch.topk(scores, 3072, dim=-1)
        torch.zeros(8, 4096).scatter_(1, ti, 1.0)
        return torch.sort(ti, dim=1)

    for name, fn in (("topk", topk), ("gather", lambda: torch.gather(xs, 1, ie)),
                     ("scatter", lambda: xs + torch.zeros_like(xs).scatter_(1, ie, ys))):
        med, n, _ = _median_time(fn, budget_s / 3)
        res["mod_" + name] = {"ms": med * 1e3, "dtype": "bf16" if name != "topk" else "fp32",
                              "sample": f"full config 4 shape, median of {n}"}
    res["host"] = host
    res["kind"] = "port"
    return res


# ----------------------------------------------------------------- config 1
def bench_c1(dev, steps=50):
    """Config 1 on the GPU: embedding (vocab 32000) * sqrt(512) then
    HydraBlock (CCGQA dim 512, 8/2 heads of 16, 4x compression, conv k=3,
    QK-mean, QK-norm, SwiGLU hidden 1365), fp32, ids [2, 512], N(0, 0.02)
    weights.  The steps are captured in one HIP graph (launch-bound
    workload: ~15 small launches), replayed untimed once, then timed."""
    import math

    from hydra_amd.layers import SwiGLUMLPFused
    from hydra_amd.model.framework import HydraBlock, embedding_lookup

    g = torch.Generator().manual_seed(0)
    with torch.device(dev):
        blk = HydraBlock(dim=512, n_heads=8, n_kv_heads=2, compression_factor=4, max_seq_len=512)
        blk.mlp = SwiGLUMLPFused(512, 1365)
        table = torch.empty(32000, 512)
    with torch.no_grad():
        for name, prm in blk.named_parameters():
            if name.endswith("key_temperature"):
                prm.fill_(4.0)
            elif "norm" in name:
                prm.fill_(1.0)
            else:
                prm.copy_(torch.randn(prm.shape, generator=g) * 0.02)
        table.copy_(torch.randn(table.shape, generator=g) * 0.02)
    blk.eval()
    ids = torch.randint(0, 32000, (2, 512), generator=g).to(dev)

    def step():
        with torch.no_grad():
            return blk(embedding_lookup(table, ids, math.sqrt(512)))

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            step()
    graph.replay()
    torch.cuda.synchronize()
    a, b = _events(2)
    a.record()
    graph.replay()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    del graph
    from oracle import blocks as ob
    from oracle import ccgqa as occ

    fl = ob.flops_c1(occ.CCGQAConfig(dim=512, n_heads=8, n_kv_heads=2, compression_factor=4), 2, 512, 1365)
    return {"value": 1024 / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms, "steps": steps,
            "dtype": "fp32", "flops": fl, "TFLOPs": fl / (ms * 1e-3) / 1e12,
            "workload": "config 1: embedding + HydraBlock, dim 512, 8/2 heads x hd 16, SwiGLU 1365, "
                        "ids [2, 512] over vocab 32000, fp32, HIP graph of the steps"}


# ----------------------------------------------------------------- config 5
def bench_c5(dev, steps=3, warmup=1):
    """Config 5: HydraModel forward at the 1B shape in bf16 -- dim 1792, 20
    MoR blocks x 4 recursions (80 effective layers), CCGQA 4x compression
    (latent 448) with the reference's 1B preset heads 28 / 4 KV (7:1; 8:1
    does not divide 448 into even head dims with a power-of-two-friendly
    layout), SwiGLU mlp_ratio 3.6 (the trainer's, hidden 6656), MoD capacity
    0.75 on the MLP of blocks 1..18 (hard routing: global step past the MoD
    warmup), MoR depth routing with the code's layer-aware router target
    0.2 -> 0.5, tied LM head over vocab 32000; ids [4, 4096]; random N(0,
    0.02) weights from the model's own init.  Eager launches; events
    bracket the K steps."""
    from hydra_amd.model.framework import HydraModel

    torch.manual_seed(0)
    with torch.device(dev):
        model = HydraModel(vocab_size=32000, dim=1792, n_mor_blocks=20, recursions_per_block=4,
                           n_heads=28, n_kv_heads=4, compression_factor=4, mlp_ratio=3.6,
                           max_seq_len=4096, mod_capacity=0.75, adaptive=True, tie_weights=True)
    model = model.to(torch.bfloat16).eval()
    model.set_global_step(10_000)
    n_params = sum(p.numel() for p in model.parameters())
    g = torch.Generator(device=dev).manual_seed(0)
    ids = torch.randint(0, 32000, (4, 4096), device=dev, generator=g)
    with torch.no_grad():
        for _ in range(warmup):
            model(ids)
        torch.cuda.synchronize()
        a, b = _events(2)
        a.record()
        for _ in range(steps):
            out = model(ids)
        b.record()
        torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    assert out.shape == (4, 4096, 32000) and torch.isfinite(out[0, :4].float()).all()
    del model, out
    torch.cuda.empty_cache()
    # one block's CCGQA prep and attention core at this shape, timed alone
    # (temperature sqrt(16) = 4, the module's initial value)
    st = C3Step(dev, B=4, S=4096, dim=1792, n_heads=28, n_kv_heads=4, comp=4, temperature=4.0)
    prep_ms, attn_ms = time_prep_and_attention(st, 40)
    fl = c3_flops(B=4, S=4096, dim=1792, Hq=28, Hkv=4, comp=4)
    prep_fl = fl["q_conv"] + fl["k_conv"]
    del st
    torch.cuda.empty_cache()
    return {"value": 4 * 4096 / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms, "steps": steps,
            "warmup": warmup, "dtype": "bf16", "params": n_params,
            "workload": "config 5: HydraModel 1B shape (dim 1792, 20 MoR blocks x 4 recursions, "
                        "28/4 heads x hd 16 (7:1, the reference's 1B preset; the config's 8:1 has no "
                        "even head dim for latent 448 with 4 kv heads), mlp 3.6, MoD 0.75 middle "
                        "blocks, MoR router target 0.2 -> 0.5 (the code's; the README's 40% -> 80% "
                        "is not in the code), vocab 32000), B4 x S4096, bf16, eager",
            "roofline": {
                "attention": {"kernel": "attn_fwd_mfma_kernel<16,causal>", "bound": "mfma",
                              "avg_ms": attn_ms, "flops_per_launch": fl["core"],
                              "achieved": fl["core"] / (attn_ms * 1e-3) / 1e12, "peak": BF16_PEAK_TFLOPS,
                              "unit": "TFLOP/s",
                              "frac": fl["core"] / (attn_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS},
                "prep": {"kernel": "ccgqa_prep_mfma_kernel<16,64>", "bound": "mfma",
                         "avg_ms": prep_ms, "flops_per_launch": prep_fl,
                         "achieved": prep_fl / (prep_ms * 1e-3) / 1e12, "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": prep_fl / (prep_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS},
            }}


def calibrate_copy(mib=512, reps=3):
    """A plain device copy of known size: under rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE, its counters give the scale between the counter readings and
    real HBM bytes (expected reading: mib*1024 KiB each way)."""
    a = torch.empty(mib << 20, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_each_way": mib << 20, "reps": reps}))


def measured_traffic(kernel_key):
    """HBM bytes per launch of a kernel from the committed PMC summary
    (profiles/traffic.json, written from rocprofv3 FETCH_SIZE + WRITE_SIZE
    passes scaled by the copy calibration); None when absent."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        return json.loads(path.read_text())["kernels"][kernel_key]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def rocpd_summary(paths, kernel_regex=None):
    """Per-kernel means from rocprofv3 result databases (rocpd SQLite): the
    number of dispatches, the mean duration, and the mean of each collected
    counter per dispatch.  Prints one block per kernel, for the profile
    summaries committed under profiles/."""
    import collections
    import re
    import sqlite3

    pat = re.compile(kernel_regex) if kernel_regex else None
    short = lambda n: re.sub(r"\(.*", "", (n or "").replace("(anonymous namespace)", "anon"))[:120]
    dur = collections.defaultdict(list)
    ctr = collections.defaultdict(lambda: collections.defaultdict(list))
    for path in paths:
        con = sqlite3.connect(path)
        views = {r[0] for r in con.execute("select name from sqlite_master where type in ('table','view')")}
        if "kernels" in views:
            cols = [r[1] for r in con.execute("pragma table_info(kernels)")]
            for row in con.execute("select * from kernels"):
                d = dict(zip(cols, row))
                name = short(d.get("name") or d.get("kernel_name"))
                if pat is None or pat.search(name):
                    dur[name].append((d["end"] - d["start"]) / 1000.0)
        if "counters_collection" in views:
            cols = [r[1] for r in con.execute("pragma table_info(counters_collection)")]
            for row in con.execute("select * from counters_collection"):
                d = dict(zip(cols, row))
                name = short(d.get("kernel_name") or d.get("name"))
                if pat is None or pat.search(name):
                    ctr[name][d["counter_name"]].append(d["value"])
    for name in sorted(set(dur) | set(ctr), key=lambda n: -sum(dur.get(n, [0]))):
        v = dur.get(name, [])
        head = f"{name}: {len(v)} dispatches"
        if v:
            head += f", mean {sum(v) / len(v):.2f} us"
        print(head)
        for cn, vals in sorted(ctr[name].items()):
            print(f"    {cn:34s} {sum(vals) / len(vals):.6g} per dispatch (n={len(vals)})")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-c3", action="store_true", help="skip every section but config 3")
    ap.add_argument("--only-attn-bwd", action="store_true",
                    help="run only the attention backward section and print its figures "
                         "(for counter runs of its kernels)")
    ap.add_argument("--no-c5", action="store_true", help="skip the config-5 model forward")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a 512 MiB device copy (traffic-counter calibration)")
    ap.add_argument("--rocpd-summary", nargs="+", metavar="DB",
                    help="summarise rocprofv3 result databases (no GPU work) and exit")
    ap.add_argument("--kernel-regex", default=None, help="with --rocpd-summary: kernels to keep")
    args = ap.parse_args()
    if args.rocpd_summary:
        rocpd_summary(args.rocpd_summary, args.kernel_regex)
        return
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the hot path has no multi-GPU "
              "component); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU", file=sys.stderr)
        sys.exit(1)
    if args.calibrate_copy:
        calibrate_copy()
        return
    from hydra_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    if args.only_attn_bwd:
        print(json.dumps({"attention_backward": bench_attention_backward(dev)}))
        return
    step, ms_step, eager_ms, stages, attn_ms = bench_c3(dev, args.steps, args.warmup)
    probe_mhz, wall_khz = shader_clock_mhz(dev)
    clock, span_ms = attention_clock(step, wall_khz)
    fl = c3_flops()
    achieved = fl["core"] / (attn_ms * 1e-3) / 1e12
    # the nominal peak is 256 CUs x 4 SIMDs x 1024 FLOP/clk at 2400 MHz
    peak_at_clock = BF16_PEAK_TFLOPS * clock / 2400.0
    line = {
        "metric": METRIC,
        "value": step.B * step.S / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seed 0, N(0,1) activations, N(0,0.02) weights)",
        "config": {"workload": "config 3: CCGQA attention forward, dim 1024, latent 256, 4q/1kv heads "
                               "x hd 64, causal conv k=3, QK-mean, QK-norm tau 1.0, B4 x S4096, bf16",
                   "global_batch": step.B, "seq_len": step.S, "parallelism": "none (1 GPU)"},
        "roofline": {"kernel": "attn_fwd_kp_kernel<64,causal>", "bound": "mfma",
                     "achieved": achieved, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / BF16_PEAK_TFLOPS,
                     "traffic": measured_traffic("attention_op<64,causal>"),
                     "flops_per_launch": fl["core"], "avg_ms": attn_ms,
                     "clock_mhz": clock, "peak_at_clock": peak_at_clock,
                     "frac_at_clock": achieved / peak_at_clock,
                     "clock_source": "the attention kernel's own s_memtime / s_memrealtime stamps "
                                     "per workgroup (5 launches after the timing)",
                     "stamped_span_ms": span_ms,
                     "probe_clock_mhz": probe_mhz},
        "launch": "HIP graph of the K steps (16 rotating 32 MiB input sets), one launch",
        "eager_ms_per_step": eager_ms,
        "stages_ms": {"eager_events": stages, "attention_graph": attn_ms},
        "module_tflops": fl["total"] / (ms_step * 1e-3) / 1e12,
    }
    if not args.only_c3:
        line["fused_ops"] = bench_fused_ops(dev)
        line["mod"] = bench_mod(dev)
        line["attention_backward"] = bench_attention_backward(dev)
        line["cross_entropy"] = bench_cross_entropy(dev)
        line["c1_block"] = bench_c1(dev)
        if not args.no_c5:
            line["c5_model"] = bench_c5(dev)
    if not args.no_cpu_baseline:
        host = host_cpu()
        line["cpu_baseline"] = cpu_baseline(host)
        if not args.only_c3:
            line["cpu_baselines"] = cpu_baselines(host)
            line["c1_block"]["cpu_tokens_per_s"] = line["cpu_baselines"]["c1_block"]["value"]
    print(json.dumps(line))


if __name__ == "__main__":
    main()
