"""CPU checks of the host-side mirror of the reference interface:
registry/factory behaviour, module structure and state_dict keys, legacy
checkpoint migration, flags, and the no-fallback rule for CPU tensors."""
from __future__ import annotations

import pytest
import torch


def test_registry():
    from hydra_amd.attention import (available_hybrid_attention_backends,
                                     is_hybrid_attention_backend_available,
                                     resolve_hybrid_attention_backend)

    assert available_hybrid_attention_backends() == ("ccqa",)
    assert resolve_hybrid_attention_backend(None).name == "ccqa"
    assert resolve_hybrid_attention_backend(" CCGQA ").name == "ccqa"
    assert is_hybrid_attention_backend_available("ccgqa")
    assert not is_hybrid_attention_backend_available("lla3")
    with pytest.raises(ValueError, match="Only 'ccgqa' is supported"):
        resolve_hybrid_attention_backend("lla3")


def test_factory_whitelist_and_env(monkeypatch):
    from hydra_amd.attention import build_hybrid_attention_module

    m = build_hybrid_attention_module("ccgqa", dim=512, n_heads=8, n_kv_heads=2, max_seq_len=64,
                                      compression_factor=4,
                                      attention_kwargs={"use_rope": False, "bogus": 1})
    assert m.use_rope is False and m.head_dim == 16
    monkeypatch.setenv("HYDRA_CCQA_USE_FUSED_KERNEL", "0")
    m = build_hybrid_attention_module("ccqa", dim=256, n_heads=4, n_kv_heads=1, max_seq_len=64,
                                      compression_factor=4, attention_kwargs={})
    assert m.use_fused_kernel is False
    with pytest.raises(ValueError):
        build_hybrid_attention_module("la3", dim=256, n_heads=4, n_kv_heads=1, max_seq_len=64,
                                      compression_factor=4, attention_kwargs={})


def test_build_ccqa_attention_both_import_paths():
    """build_ccqa_attention from the package (backends/ccgqa/__init__.py:12-15,
    a lazy alias) and from backend.py (:8-17) build the same module."""
    from hydra_amd.attention import CCGQAAttention
    from hydra_amd.attention.backends.ccgqa import build_ccqa_attention as from_pkg
    from hydra_amd.attention.backends.ccgqa.backend import build_ccqa_attention as from_backend

    kw = dict(dim=256, n_heads=4, n_kv_heads=1, compression_factor=4, max_seq_len=64, conv_kernel_size=5)
    a, b = from_pkg(**kw), from_backend(**kw)
    assert type(a) is CCGQAAttention and type(b) is CCGQAAttention
    assert a.conv_kernel_size == 5 and a.q_conv.kernel_size == 5
    assert a.state_dict().keys() == b.state_dict().keys()


def test_module_structure_matches_reference():
    """Paper-compliance structure of the debug shape (tests/test_paper_compliance.py:185-272)."""
    from hydra_amd.attention import CCGQAAttention

    m = CCGQAAttention(dim=512, n_heads=8, n_kv_heads=2, compression_factor=4, max_seq_len=64)
    assert m.latent_dim == 128 and m.head_dim == 16 and m.kv_dim == 32
    assert m.qkv_proj.out_features == 128 + 2 * 32
    assert tuple(m.q_conv.conv1.weight.shape) == (128, 16, 3)
    assert tuple(m.q_conv.conv2.weight.shape) == (128, 128, 3)
    assert tuple(m.k_conv.conv1.weight.shape) == (32, 16, 3)
    assert tuple(m.k_conv.conv2.weight.shape) == (32, 32, 3)
    assert m.key_temperature.requires_grad and m.key_temperature.item() == pytest.approx(4.0)
    assert sorted(m.state_dict()) == sorted([
        "qkv_proj.weight", "o_proj.weight", "q_conv.conv1.weight", "q_conv.conv2.weight",
        "k_conv.conv1.weight", "k_conv.conv2.weight", "key_temperature"])
    assert tuple(m.cos_cached.shape) == (1, 1, 64, 8)
    with pytest.raises(AssertionError):
        CCGQAAttention(dim=96, n_heads=16, n_kv_heads=4, compression_factor=2)  # hd = 3, odd


def test_legacy_state_dict_migration():
    from hydra_amd.attention import CCGQAAttention

    m = CCGQAAttention(dim=256, n_heads=4, n_kv_heads=1, compression_factor=4, max_seq_len=16)
    sd = m.state_dict()
    L, K = m.latent_dim, m.kv_dim
    W = sd.pop("qkv_proj.weight")
    legacy = dict(sd)
    legacy["q_down.weight"] = W[:L]
    legacy["k_down.weight"] = W[L:L + K]
    legacy["v_down.weight"] = W[L + K:L + K + K // 2]
    legacy["v_shift_down.weight"] = W[L + K + K // 2:]
    legacy["q_conv1.weight"] = legacy.pop("q_conv.conv1.weight")
    m2 = CCGQAAttention(dim=256, n_heads=4, n_kv_heads=1, compression_factor=4, max_seq_len=16)
    m2.load_state_dict(legacy)
    assert torch.equal(m2.qkv_proj.weight, W)
    assert torch.equal(m2.q_conv.conv1.weight, m.q_conv.conv1.weight)


def test_kernel_flags_and_disable():
    import hydra_amd.kernels.fused_ops as fo

    st = fo.get_kernel_status()
    for key in ("triton_available", "use_triton_kernels", "fused_rope", "fused_qk_norm",
                "fused_swiglu", "fused_rms_norm"):
        assert key in st
    try:
        fo.set_use_triton_kernels(False)
        with pytest.raises(RuntimeError, match="disabled"):
            fo.fused_swiglu(torch.randn(4), torch.randn(4))
    finally:
        fo.set_use_triton_kernels(True)


def test_cpu_tensors_raise_not_fallback():
    from hydra_amd.attention import CCGQAAttention
    from hydra_amd.kernels import fused_rms_norm, fused_rope, fused_swiglu
    from hydra_amd.routing import gather_by_indices, mod_topk

    with pytest.raises(RuntimeError, match="GPU tensors only"):
        fused_rms_norm(torch.randn(2, 8), torch.ones(8))
    with pytest.raises(RuntimeError, match="GPU tensors only"):
        fused_swiglu(torch.randn(2, 8), torch.randn(2, 8))
    with pytest.raises(RuntimeError, match="GPU tensors only"):
        fused_rope(torch.randn(1, 1, 4, 8), torch.randn(4, 4), torch.randn(4, 4))
    with pytest.raises(RuntimeError, match="GPU tensors only"):
        mod_topk(torch.randn(2, 8), 3)
    with pytest.raises(RuntimeError, match="GPU tensors only"):
        gather_by_indices(torch.randn(1, 8, 4), torch.zeros(1, 2, dtype=torch.long))
    m = CCGQAAttention(dim=256, n_heads=4, n_kv_heads=1, compression_factor=4, max_seq_len=16)
    with pytest.raises(RuntimeError, match="GPU tensors only"):
        m(torch.randn(1, 8, 256))


def test_capacity_k():
    from hydra_amd.routing import compute_capacity_k, router_k

    assert router_k(4096, 0.75) == 3072
    assert router_k(10, 0.0) == 1 and router_k(10, 2.0) == 10
    assert compute_capacity_k(512, 0.5) == 256 and compute_capacity_k(3, 0.1) == 1
