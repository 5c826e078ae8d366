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
    (fused_ops.py:1251-1281), whose grad_x no closed form pins;
  * ChunkedCrossEntropyFunction's target clamping (fused_ops.py:1407-1422);
  * the config-1 block composition (embedding lookup + HydraBlock) and a
    small HydraModel (MoR blocks, MoD, tied LM head) saved through the
    reference's own save_checkpoint, with its forward output.

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


def make_chunked_ce() -> None:
    """ChunkedCrossEntropyFunction (hydra/kernels/fused_ops.py:1382-1531) on
    targets that mix ignore_index entries with out-of-range ones, where the
    reference clamps the whole target vector (:1407-1422) and the clamped
    ignore entries then count as valid; and a case with ignore entries only."""
    from hydra.kernels.fused_ops import ChunkedCrossEntropyFunction

    g = torch.Generator().manual_seed(13)
    B, L, D, V = 2, 24, 32, 100
    h = bf16_round(torch.randn(B, L, D, generator=g))
    w = bf16_round(torch.randn(V, D, generator=g) * 0.3)
    arrays = {"h": bf16_bits(h), "w": bf16_bits(w)}
    for name, oob in (("mixed", True), ("ignore_only", False)):
        t = torch.randint(0, V, (B, L), generator=g)
        t[0, 2], t[1, 5], t[1, 6] = -100, -100, -100
        if oob:
            t[0, 7], t[1, 11] = 130, -4
        hh, ww = h.clone().requires_grad_(), w.clone().requires_grad_()
        loss = ChunkedCrossEntropyFunction.apply(hh, ww, t, -100, 16)
        (loss * 0.7).backward()
        arrays.update({f"{name}_targets": t.numpy(), f"{name}_loss": loss.detach().numpy(),
                       f"{name}_grad_h": hh.grad.numpy(), f"{name}_grad_w": ww.grad.numpy()})
    arrays["grad_output"] = np.array(0.7)
    np.savez_compressed(HERE / "chunked_ce_cpu.npz", **arrays)
    print("wrote chunked ce")


def _bf16_init_(module: torch.nn.Module, g: torch.Generator, std: float = 0.02) -> dict:
    """Overwrite every parameter with bf16-representable N(0, std) values
    (norm gains N(1, 0.1), the key temperature kept at its init, rounded);
    returns {name: bf16 bits}."""
    arrays = {}
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.endswith("key_temperature"):
                p.copy_(bf16_round(p))
            elif name.endswith("norm1.weight") or name.endswith("norm2.weight") or name.endswith("norm.weight"):
                p.copy_(bf16_round(1.0 + 0.1 * torch.randn(p.shape, generator=g)))
            elif name.endswith("router.bias"):
                p.copy_(bf16_round(p))
            else:
                p.copy_(bf16_round(torch.randn(p.shape, generator=g) * std))
            arrays["w." + name] = bf16_bits(p)
    return arrays


def make_hydra_block() -> None:
    """Config-1 composition: _safe_embedding_lookup
    (hydra/model/framework/model.py:51-73, scale sqrt(dim), ids clamped) then
    HydraBlock.forward (blocks.py:68-70) with its MLP replaced by
    SwiGLUMLPFused(dim, int(dim * 8/3)) (the unrounded hidden of config 1),
    fp32 on the CPU.  Reduced shape: dim 256 with compression 2 keeps config
    1's head layout (8 query / 2 KV heads of 16); vocab 512 with two
    out-of-range ids; B 2 x S 40."""
    import math

    from hydra.layers import SwiGLUMLPFused
    from hydra.model.framework.blocks import HydraBlock
    from hydra.model.framework.model import _safe_embedding_lookup

    torch.manual_seed(3000)
    dim, vocab, hidden = 256, 512, int(256 * 8 / 3)
    blk = HydraBlock(dim=dim, n_heads=8, n_kv_heads=2, compression_factor=2, max_seq_len=64).eval()
    blk.mlp = SwiGLUMLPFused(dim, hidden)
    emb = torch.nn.Embedding(vocab, dim)
    g = torch.Generator().manual_seed(3001)
    arrays = _bf16_init_(blk, g)
    with torch.no_grad():
        emb.weight.copy_(bf16_round(torch.randn(vocab, dim, generator=g) * 0.02))
        ids = torch.randint(0, vocab, (2, 40), generator=g)
        ids[0, 5], ids[1, 17] = vocab + 9, -2  # clamped by the lookup
        h0 = _safe_embedding_lookup(emb, ids, scale=math.sqrt(dim))
        out = blk(h0)
    arrays.update({"w.tok_emb.weight": bf16_bits(emb.weight), "ids": ids.numpy(),
                   "h0": h0.numpy(), "out": out.numpy().astype(np.float32),
                   "meta": np.array(repr(dict(dim=dim, vocab=vocab, hidden=hidden, n_heads=8,
                                              n_kv_heads=2, compression_factor=2)))})
    np.savez_compressed(HERE / "hydra_block_c1.npz", **arrays)
    print("wrote hydra block", out.shape)


def _import_reference_checkpointing():
    """hydra.training's package __init__ imports the trainer, which needs
    hydra.data (absent from the reference tree); checkpointing.py itself
    needs only .config and .metrics.  Register the package by path without
    running its __init__, then import the three real modules."""
    import importlib
    import types

    if "hydra.training" not in sys.modules:
        import hydra

        pkg = types.ModuleType("hydra.training")
        pkg.__path__ = [str(Path(hydra.__file__).parent / "training")]
        sys.modules["hydra.training"] = pkg
    ck = importlib.import_module("hydra.training.checkpointing")
    cfg = importlib.import_module("hydra.training.config")
    met = importlib.import_module("hydra.training.metrics")
    return ck, cfg, met


def make_hydra_model() -> None:
    """A small HydraModel (hydra/model/framework/model.py:166-515) in the
    reference's own checkpoint format: save_checkpoint
    (hydra/training/checkpointing.py:99-192) writes the file, and the
    model's eval forward on token ids (MoD enabled in the middle block,
    adaptive MoR, tied LM head) is stored beside it.  fp32 on the CPU."""
    import logging

    from hydra.model.framework.model import HydraModel

    ck, cfgm, met = _import_reference_checkpointing()
    torch.manual_seed(4000)
    model = HydraModel(vocab_size=256, dim=128, n_mor_blocks=3, recursions_per_block=3, n_heads=4,
                       n_kv_heads=1, compression_factor=2, mlp_ratio=2.0, max_seq_len=64,
                       mod_capacity=0.75, adaptive=True, tie_weights=True)
    g = torch.Generator().manual_seed(4001)
    _bf16_init_(model, g)
    with torch.no_grad():  # MoR router weights wide enough that depths vary per token
        for layer in model.layers:
            w = layer.mor_router.router.weight
            w.copy_(bf16_round(torch.randn(w.shape, generator=g) * 0.5))
    model.set_global_step(10_000)  # past the MoD warmup: hard routing in the middle block
    model.eval()
    with torch.no_grad():
        ids = torch.randint(0, 256, (2, 40), generator=g)
        logits = model(ids)
        hidden = model.forward_hidden(ids)
    cdir = HERE / "_ckpt"
    cdir.mkdir(exist_ok=True)
    cfg = cfgm.TrainingConfig()
    cfg.checkpoint_dir = str(cdir)
    cfg.model_size = "golden"
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    scaler = torch.amp.GradScaler("cpu", enabled=False)
    metrics = met.TrainingMetrics()
    path = ck.save_checkpoint(step=7, config=cfg, model=model, optimizer=opt, scaler=scaler,
                              metrics=metrics, checkpoint_history=[], final=True,
                              logger=logging.getLogger("make_golden"))
    dst = HERE / "hydra_model_ckpt.pt"
    Path(path).replace(dst)
    cdir.rmdir()
    np.savez_compressed(HERE / "hydra_model_fwd.npz", ids=ids.numpy(),
                        logits=logits.numpy().astype(np.float32),
                        hidden=hidden.numpy().astype(np.float32),
                        meta=np.array(repr(dict(vocab_size=256, dim=128, n_mor_blocks=3,
                                                recursions_per_block=3, n_heads=4, n_kv_heads=1,
                                                compression_factor=2, mlp_ratio=2.0, max_seq_len=64,
                                                mod_capacity=0.75, global_step=10_000))))
    print("wrote hydra model", logits.shape, dst.stat().st_size, "bytes")


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
    make_chunked_ce()
    make_hydra_block()
    make_hydra_model()
    (HERE / "VERSIONS.txt").write_text(
        f"torch {torch.__version__}\nnumpy {np.__version__}\nreference {ref} (hydra 0.2.0)\n"
    )


if __name__ == "__main__":
    main()
