"""Reference checkpoint files (hydra/training/checkpointing.py:134-150) load
into the hot-path modules: the dict layout, torch.compile's "_orig_mod."
prefix, a submodule prefix, and CCGQAAttention's legacy-key migration
(attention.py:333-383).  CPU only: no kernel runs."""
from __future__ import annotations

import pytest
import torch

from hydra_amd.attention import CCGQAAttention
from hydra_amd.training import load_module_from_checkpoint, module_state, read_checkpoint


def _attn():
    torch.manual_seed(0)
    return CCGQAAttention(dim=256, n_heads=4, n_kv_heads=2, compression_factor=4, max_seq_len=64)


def _ckpt(state, prefix):
    return {"step": 7, "model": {prefix + k: v for k, v in state.items()},
            "optimizer": {"state": {}, "param_groups": []}, "scaler": {}, "config": {"lr": 1e-3},
            "metrics": {"best_loss": 2.5, "total_tokens": 1024}}


def test_load_attention_from_reference_checkpoint(tmp_path):
    src = _attn()
    with torch.no_grad():
        for p in src.parameters():
            p.normal_()
    path = tmp_path / "hydra_debug_step_7.pt"
    torch.save(_ckpt(src.state_dict(), "_orig_mod.blocks.2.attention."), path)
    dst = _attn()
    load_module_from_checkpoint(dst, path, prefix="blocks.2.attention.")
    for (k, a), (_, b) in zip(src.state_dict().items(), dst.state_dict().items()):
        assert torch.equal(a, b), k
    assert read_checkpoint(path)["step"] == 7


def test_legacy_keys_migrate_through_checkpoint():
    src = _attn()
    sd = src.state_dict()
    legacy = {}
    for k, v in sd.items():
        legacy[k.replace("q_conv.conv1", "q_conv1").replace("k_conv.conv2", "k_conv2")] = v
    qkv = legacy.pop("qkv_proj.weight")
    qr, kvr = src.n_heads * src.head_dim, src.n_kv_heads * src.head_dim
    # with value shift the v rows are v_down | v_shift_down, half each
    sizes = [qr, kvr] + ([kvr // 2, kvr - kvr // 2] if src.use_value_shift else [kvr])
    parts = torch.split(qkv, sizes, dim=0)
    for name, t in zip(("q_down", "k_down", "v_down", "v_shift_down"), parts):
        legacy[name + ".weight"] = t
    dst = _attn()
    load_module_from_checkpoint(dst, _ckpt(legacy, "model.attn."), prefix="model.attn.")
    for k2, a in sd.items():
        assert torch.equal(a, dst.state_dict()[k2]), k2


class _Custom:
    pass


def test_missing_prefix_and_unsafe_file(tmp_path):
    with pytest.raises(KeyError):
        module_state({"model": {"a.weight": torch.zeros(1)}}, "b.")
    path = tmp_path / "unsafe.pt"
    torch.save({"model": {}, "obj": _Custom()}, path)
    with pytest.raises(RuntimeError, match="weights_only"):
        read_checkpoint(path)
