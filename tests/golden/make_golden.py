"""Write the golden vectors under tests/golden/ by running the reference
(mcpirate17/HYDRA, read-only at /root/reference) on the CPU.

Only this script touches the reference; the fixtures it writes are plain
arrays (inputs, weights, expected outputs) in .npz files.  It is run by hand
in the build container, never by the tests and never on a GPU box:

    python tests/golden/make_golden.py [--ref /root/reference]

What it pins (functions whose composition no closed form fixes):
  * CCGQAAttention.forward (hydra/attention/backends/ccgqa/attention.py:201-331)
    at several head layouts and feature switches, fp32, with and without a
    padding mask;
  * MoDRouter.forward (hydra/routing/mixture_of_depths.py:159-216): k, the
    top-k indices and the mask, on scores with forced ties, plus whether
    torch.topk itself resolves those ties to the lowest index;
  * the CPU fallbacks of the fused ops (hydra/kernels/fused_ops.py:300-306,
    587-596, 881-883, 1196-1205) and the RMSNorm backward
    (fused_ops.py:1251-1281), whose grad_x no closed form pins.

All weights and inputs are rounded to bf16-representable values and stored as
raw bf16 bit patterns (uint16), so the fp32 and bf16 device paths see the
exact same inputs; expected outputs are fp32.
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bf16_round(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


CCGQA_CASES = [
    # name, ctor kwargs, (B, S), temperature, use padding mask
    ("debug_gqa4_hd16", dict(dim=512, n_heads=8, n_kv_heads=2, compression_factor=4), (2, 48), None, False),
    ("c3_gqa4_hd64", dict(dim=512, n_heads=4, n_kv_heads=1, compression_factor=2), (1, 40), 1.0, False),
    ("mha_hd32", dict(dim=256, n_heads=4, n_kv_heads=4, compression_factor=2), (2, 37), None, False),
    ("gqa2_hd32_mask", dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=2), (2, 33), 0.5, True),
    ("noconv_nomean_hd16", dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4,
                                use_convs=False, use_qk_mean=False), (1, 24), None, False),
    ("nonorm_norope_novshift_hd16", dict(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4,
                                         use_qk_norm=False, use_rope=False, use_value_shift=False),
     (1, 24), None, False),
]


def make_ccgqa(ref_root: Path) -> None:
    from hydra.attention.backends.ccgqa.attention import CCGQAAttention

    for i, (name, kw, (B, S), temp, use_mask) in enumerate(CCGQA_CASES):
        torch.manual_seed(1000 + i)
        attn = CCGQAAttention(max_seq_len=128, **kw).eval()
        g = torch.Generator().manual_seed(2000 + i)
        arrays = {}
        with torch.no_grad():
            for pname, p in attn.named_parameters():
                if pname == "key_temperature":
                    if temp is not None:
                        p.fill_(temp)
                    p.copy_(bf16_round(p))
                else:
                    p.copy_(bf16_round(torch.randn(p.shape, generator=g) * 0.02))
                arrays["w." + pname] = bf16_bits(p)
            x = bf16_round(torch.randn(B, S, kw["dim"], generator=g))
            mask = None
            if use_mask:
                mask = (torch.rand(B, S, generator=g) > 0.25).to(torch.int64)
                mask[:, 0] = 1  # every query keeps at least one visible key
                arrays["mask"] = mask.numpy().astype(np.uint8)
            out = attn(x, mask=mask)
        arrays["x"] = bf16_bits(x)
        arrays["out"] = out.numpy().astype(np.float32)
        meta = dict(kw)
        meta.update(B=B, S=S, max_seq_len=128)
        arrays["meta"] = np.array(repr(sorted(meta.items())))
        np.savez_compressed(HERE / f"ccgqa_{name}.npz", **arrays)
        print("wrote", name, out.shape)


def make_mod() -> None:
    from hydra.routing.mixture_of_depths import MoDRouter

    B, L, D = 4, 256, 64
    g = torch.Generator().manual_seed(7)
    for cap in (0.75, 0.5, 0.125):
        router = MoDRouter(dim=D, capacity_ratio=cap).eval()
        with torch.no_grad():
            router.router.weight.copy_(bf16_round(torch.randn(1, D, generator=g) * 0.02))
            router.router.bias.copy_(bf16_round(router.router.bias))
            x = bf16_round(torch.randn(B, L, D, generator=g))
            # Force ties: copy whole token rows so their scores are identical.
            for b in range(B):
                src = torch.randint(0, L, (L // 8,), generator=g)
                dst = torch.randint(0, L, (L // 8,), generator=g)
                x[b, dst] = x[b, src]
            mask, idx, scores = router(x, return_scores=True)
        order = torch.sort(scores, dim=-1, descending=True, stable=True).indices[:, : idx.shape[1]]
        tag = f"{int(cap * 1000):04d}"
        np.savez_compressed(
            HERE / f"mod_router_cap{tag}.npz",
            x=bf16_bits(x),
            w=bf16_bits(router.router.weight),
            b=bf16_bits(router.router.bias),
            scores=scores.numpy().astype(np.float32),
            mask=mask.numpy().astype(np.float32),
            indices=idx.numpy().astype(np.int64),
            stable_order=order.numpy().astype(np.int64),
            topk_matches_stable=np.array(bool(torch.equal(order, idx))),
            capacity_ratio=np.array(cap),
        )
        print("wrote mod cap", cap, "k =", idx.shape[1], "topk==stable:", torch.equal(order, idx))


def make_fused_ops() -> None:
    import hydra.kernels.fused_ops as fo

    g = torch.Generator().manual_seed(11)
    x = bf16_round(torch.randn(3, 5, 96, generator=g))
    w = bf16_round(1.0 + 0.1 * torch.randn(96, generator=g))
    gate = bf16_round(torch.randn(4, 7, 40, generator=g) * 3)
    up = bf16_round(torch.randn(4, 7, 40, generator=g))
    xr = bf16_round(torch.randn(2, 3, 20, 16, generator=g))
    freqs = 1.0 / (10000.0 ** (torch.arange(0, 16, 2).float() / 16))
    ang = torch.outer(torch.arange(20, dtype=torch.float32), freqs)
    cos, sin = ang.cos()[None, None], ang.sin()[None, None]
    q = bf16_round(torch.randn(2, 4, 9, 16, generator=g))
    k = bf16_round(torch.randn(2, 2, 9, 16, generator=g))
    with torch.no_grad():
        np.savez_compressed(
            HERE / "fused_ops_cpu.npz",
            x=bf16_bits(x), w=bf16_bits(w), eps=np.array(1e-6),
            rms_out=fo._rms_norm_pytorch(x, w, 1e-6).numpy(),
            gate=bf16_bits(gate), up=bf16_bits(up),
            swiglu_out=fo._swiglu_pytorch(gate, up).numpy(),
            xr=bf16_bits(xr), cos=cos.numpy(), sin=sin.numpy(),
            rope_out=fo._rope_pytorch(xr, cos, sin).numpy(),
            q=bf16_bits(q), k=bf16_bits(k), scale=np.array(8.0), temperature=np.array(0.75),
            qn_out=fo._qk_norm_pytorch(q, k, 8.0, 0.75)[0].numpy(),
            kn_out=fo._qk_norm_pytorch(q, k, 8.0, 0.75)[1].numpy(),
        )
    print("wrote fused ops")


def make_fused_ops_backward() -> None:
    """_rms_norm_backward_pytorch (hydra/kernels/fused_ops.py:1251-1281): its
    grad_x correction term is not the exact derivative, so no autograd check
    pins it; these vectors do.  Rows of x are scaled so mean(x^2) spans ~0.04
    to ~25 (the term's missing factor is visible), plus rows large enough
    for the +-100 clamp."""
    import hydra.kernels.fused_ops as fo

    g = torch.Generator().manual_seed(12)
    rows, dim = 24, 80
    scales = torch.cat([torch.full((8,), 0.2), torch.full((8,), 1.0), torch.full((6,), 5.0),
                        torch.full((2,), 40.0)])
    x = bf16_round(torch.randn(rows, dim, generator=g) * scales[:, None])
    w = bf16_round(torch.randn(dim, generator=g))
    go = bf16_round(torch.randn(rows, dim, generator=g) * 3.0)
    go[-1] = bf16_round(torch.full((dim,), 900.0))  # a clamped row
    with torch.no_grad():
        gx, gw, _ = fo._rms_norm_backward_pytorch(x, w, go, 1e-6, x.shape)
        np.savez_compressed(
            HERE / "fused_ops_bwd_cpu.npz",
            x=bf16_bits(x), w=bf16_bits(w), grad_out=bf16_bits(go), eps=np.array(1e-6),
            rms_grad_x=gx.numpy(), rms_grad_w=gw.numpy(),
        )
    print("wrote fused ops backward")


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()
    ref = Path(args.ref)
    sys.path.insert(0, str(ref))
    torch.set_num_threads(4)
    make_ccgqa(ref)
    make_mod()
    make_fused_ops()
    make_fused_ops_backward()
    (HERE / "VERSIONS.txt").write_text(
        f"torch {torch.__version__}\nnumpy {np.__version__}\nreference {ref} (hydra 0.2.0)\n"
    )


if __name__ == "__main__":
    main()
