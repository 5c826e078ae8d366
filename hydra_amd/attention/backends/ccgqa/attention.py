"""CCGQAAttention on MI355X: drop-in for
hydra/attention/backends/ccgqa/attention.py:67-383.

Same constructor, attributes, parameters and state_dict keys
(qkv_proj.weight, o_proj.weight, q_conv.conv1.weight, q_conv.conv2.weight,
k_conv.conv1.weight, k_conv.conv2.weight, key_temperature) and the same
non-persistent RoPE buffers (cos_cached, sin_cached).  The forward is

    qkv  = x @ W_qkv^T                              torch GEMM (hipBLASLt)
    q,k,v = hydra_ccgqa_prep_fwd(qkv, ...)          one HIP kernel: split, value
                                                    shift, convs, QK-mean,
                                                    L2-norm * temperature, RoPE
    o    = hydra_attn_fwd(q, k, v, causal)          one HIP kernel (bf16 MFMA),
                                                    written as [B, S, L]
    out  = o @ W_o^T * output_scale                 torch GEMM

With autograd recording the forward goes through CCGQAPrepFunction and
CCGQAAttentionFused (MaskedAttentionFunction with a padding mask) instead,
whose backwards are the HIP prep backward (plus the convs' GEMMs) and the
HIP attention backward; in eval() mode with grad-enabled parameters the
inference kernels run and a backward recomputes the training path.

The reference's precomputed [max_seq_len, max_seq_len] causal mask buffer is
not kept: the kernel derives causality from indices.
"""
from __future__ import annotations

import os
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from ...._lib import CCGQA_V_TRANSPOSED, CCGQA_W_TILED, MASK_KEY_PADDING, MASK_REFERENCE_SDPA
from .autograd import ccgqa_prep_train
from .kernels.fused_attention import CCGQAAttentionFused, MaskedAttentionFunction
from .kernels.fused_conv import OptimizedConvSequence
from .ops import (attention_forward, ccgqa_prep, linear_weight_ok, output_projection, pack_conv_weight,
                  pack_linear_weight, prep_flags, tiled_weights_ok)

# Kept for callers that probe these names (attention.py:13-28).
FUSED_KERNELS_AVAILABLE = True
TRITON_ATTENTION_AVAILABLE = True


def _mask_mode() -> int:
    """How a padding mask passed to forward() is applied.

    "reference" (default) reproduces attention.py:268-299 literally, including
    its hand-off of a "True = masked" boolean to SDPA (which reads True as
    "attend"); "key_padding" applies the mask as a key-padding mask on top of
    causality."""
    v = os.environ.get("HYDRA_CCGQA_MASK_SEMANTICS", "reference").strip().lower()
    return MASK_KEY_PADDING if v in {"key_padding", "padding"} else MASK_REFERENCE_SDPA


class _EvalRecompute(torch.autograd.Function):
    """CCGQAAttention in eval() mode with autograd recording (parameters
    that require grad, an input that does not): the forward runs the
    inference kernels and keeps only x; the backward runs the training path
    (CCGQAPrepFunction, CCGQAAttentionFused, F.linear) on x again and
    differentiates that.  Its gradients are those of the training path,
    whose forward equals the inference forward within bf16 rounding."""

    @staticmethod
    def forward(ctx, module, x, mask, *params):
        ctx.module = module
        ctx.mask = mask
        ctx.save_for_backward(x)
        qkv = F.linear(x, module.qkv_proj.weight)
        flags, convw = module._prep_args()
        return module._forward_infer(x, qkv, flags, convw, mask)

    @staticmethod
    def backward(ctx, grad_out):
        (x,) = ctx.saved_tensors
        m = ctx.module
        params = tuple(m.parameters())
        with torch.enable_grad():
            xr = x.detach().requires_grad_(ctx.needs_input_grad[1])
            qkv = F.linear(xr, m.qkv_proj.weight)
            flags, convw = m._prep_args()
            out = m._forward_train(qkv, flags, convw, ctx.mask)
            wrt = ([xr] if xr.requires_grad else []) + [p for p in params if p.requires_grad]
            grads = list(torch.autograd.grad(out, wrt, grad_out, allow_unused=True))
        dx = grads.pop(0) if xr.requires_grad else None
        dparams = [grads.pop(0) if p.requires_grad else None for p in params]
        return (None, dx, None, *dparams)


class CCGQAAttention(nn.Module):
    """Compressed Convolutional Grouped Query Attention on gfx950."""

    def __init__(self, dim: int, n_heads: int = 16, n_kv_heads: int = 4,
                 compression_factor: int = 4, max_seq_len: int = 8192, use_rope: bool = True,
                 use_qk_norm: bool = True, use_convs: bool = True, use_qk_mean: bool = True,
                 use_value_shift: bool = True, conv_kernel_size: int = 3,
                 use_fused_kernel: bool = True):
        super().__init__()
        self.dim = dim
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.n_groups = n_heads // n_kv_heads
        self.compression_factor = compression_factor
        self.use_rope = use_rope
        self.use_qk_norm = use_qk_norm
        self.use_convs = use_convs
        self.use_qk_mean = use_qk_mean
        self.use_value_shift = use_value_shift
        self.use_fused_kernel = use_fused_kernel
        self.conv_kernel_size = conv_kernel_size

        self.latent_dim = dim // compression_factor
        self.head_dim = self.latent_dim // n_heads
        self.kv_dim = n_kv_heads * self.head_dim
        assert self.latent_dim % n_heads == 0, (
            f"latent_dim {self.latent_dim} must be divisible by n_heads {n_heads}")
        assert self.head_dim % 2 == 0, (
            f"head_dim {self.head_dim} must be even for RoPE (splits into pairs)")

        # q | k | v_curr | v_prev  (or q | k | v without the value shift)
        self.qkv_proj = nn.Linear(dim, self.latent_dim + 2 * self.kv_dim, bias=False)
        self.o_proj = nn.Linear(self.latent_dim, dim, bias=False)
        self.output_scale = float(os.environ.get("HYDRA_CCGQA_OUTPUT_SCALE", "1.0"))
        if use_convs:
            self.q_conv = OptimizedConvSequence(self.latent_dim, n_heads, 1, conv_kernel_size)
            self.k_conv = OptimizedConvSequence(self.kv_dim, n_kv_heads, 1, conv_kernel_size)
        self.key_temperature = nn.Parameter(torch.full((1,), float(self.head_dim ** 0.5)))
        if use_rope:
            self._init_rope(max_seq_len)
        self.scale = self.head_dim ** -0.5
        self.max_seq_len = max_seq_len

    def _init_rope(self, max_seq_len: int) -> None:
        """attention.py:160-185 (theta 1e4, fp32 unless HYDRA_ROPE_CACHE_DTYPE)."""
        hd = self.head_dim
        freqs = 1.0 / (10000.0 ** (torch.arange(0, hd, 2).float() / hd))
        ang = torch.outer(torch.arange(max_seq_len, dtype=torch.float32), freqs)
        env = os.environ.get("HYDRA_ROPE_CACHE_DTYPE", "").strip().lower()
        cdt = {"bf16": torch.bfloat16, "bfloat16": torch.bfloat16, "fp16": torch.float16,
               "float16": torch.float16, "half": torch.float16}.get(env, torch.float32)
        self.register_buffer("cos_cached", ang.cos().to(cdt)[None, None], persistent=False)
        self.register_buffer("sin_cached", ang.sin().to(cdt)[None, None], persistent=False)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, S, _ = x.shape
        if self.use_rope and S > self.cos_cached.shape[2]:
            raise ValueError(f"CCGQAAttention: sequence length {S} exceeds the RoPE cache "
                             f"({self.cos_cached.shape[2]})")
        recording = torch.is_grad_enabled() and (
            x.requires_grad or any(p.requires_grad for p in self.parameters()))
        if recording and not (self.training or x.requires_grad):
            # eval() with parameters that require grad: the inference kernels
            # give the output; a backward, if one comes, recomputes the
            # forward through the training path (as activation checkpointing
            # would) instead of keeping its activations now.
            return _EvalRecompute.apply(self, x, mask, *self.parameters())
        qkv = F.linear(x, self.qkv_proj.weight)
        flags, convw = self._prep_args()
        if recording:
            return self._forward_train(qkv, flags, convw, mask)
        return self._forward_infer(x, qkv, flags, convw, mask)

    def _prep_args(self):
        """The prep kernel's feature flags and the four conv weights (Conv1d
        layout; empty without convs)."""
        flags = prep_flags(self.use_convs, self.use_qk_mean, self.use_value_shift,
                           self.use_qk_norm, self.use_rope)
        convw = ((self.q_conv.conv1.weight, self.q_conv.conv2.weight,
                  self.k_conv.conv1.weight, self.k_conv.conv2.weight)
                 if self.use_convs else ())
        return flags, convw

    def _forward_infer(self, x, qkv, flags, convw, mask):
        """The inference kernels: prep with V^T rows and MFMA-tiled conv
        weights, the attention kernel writing [B, S, L], o_proj in
        hydra_linear_fwd."""
        B, S, _ = x.shape
        if x.dtype == torch.bfloat16 and S % 8 == 0 and self.head_dim in (16, 32, 64, 128):
            flags |= CCGQA_V_TRANSPOSED  # V^T feeds the MFMA attention without a transpose
        tiled = (self.use_convs and self.conv_kernel_size == 3 and
                 tiled_weights_ok(self.n_heads, self.n_kv_heads, self.head_dim, x.dtype))
        if tiled:
            flags |= CCGQA_W_TILED  # conv weights in MFMA-fragment order
        with torch.no_grad():
            packed = self._packed_conv_weights(convw, x.dtype, tiled) if self.use_convs else (None,) * 4
            q, k, v = ccgqa_prep(
                qkv.detach(), self.n_heads, self.n_kv_heads, self.head_dim, flags, *packed,
                temperature=self.key_temperature if self.use_qk_norm else None,
                cos=self.cos_cached if self.use_rope else None,
                sin=self.sin_cached if self.use_rope else None, packed=True,
                conv_ks=self.conv_kernel_size)
            out = torch.empty((B, S, self.latent_dim), dtype=x.dtype, device=x.device)
            o_view = out.view(B, S, self.n_heads, self.head_dim).transpose(1, 2)
            attention_forward(q, k, v, causal=True, scale=self.scale,
                              key_mask=mask, mask_mode=_mask_mode() if mask is not None else 0,
                              out=o_view,
                              bound_temperature=self.key_temperature if self.use_qk_norm else None)
        w_o = self.o_proj.weight
        out = output_projection(out, w_o, self._packed_o_proj() if linear_weight_ok(w_o) else None)
        if self.output_scale != 1.0:
            out = out * self.output_scale
        return out

    def _forward_train(self, qkv: torch.Tensor, flags: int, convw, mask=None) -> torch.Tensor:
        """The forward with autograd: CCGQAPrepFunction (prep kernel forward;
        pointwise backward kernel plus the convs' backward as GEMMs), then
        CCGQAAttentionFused (the HIP attention forward and backward) or, with
        a padding mask, MaskedAttentionFunction (the same kernels with the
        key mask), as the reference trains attention.py:201-331 through
        autograd."""
        B, S, _ = qkv.shape
        w = tuple(convw) if self.use_convs else (None,) * 4
        q, k, v = ccgqa_prep_train(
            qkv, self.n_heads, self.n_kv_heads, self.head_dim, flags, *w,
            temperature=self.key_temperature if self.use_qk_norm else None,
            cos=self.cos_cached if self.use_rope else None,
            sin=self.sin_cached if self.use_rope else None)
        if mask is None:
            o = CCGQAAttentionFused.apply(q, k, v, True, True)
        else:
            o = MaskedAttentionFunction.apply(q, k, v, mask.to(q.device), _mask_mode(), True)
        out = F.linear(o.transpose(1, 2).reshape(B, S, self.latent_dim), self.o_proj.weight)
        if self.output_scale != 1.0:
            out = out * self.output_scale
        return out

    def _packed_conv_weights(self, convw, dtype, tiled=False):
        """Packed copies (tap-major, or MFMA-tiled) of the four conv weights in
        `dtype`, rebuilt only when a weight changes (tensor version counter)
        or moves."""
        key = tuple((w.data_ptr(), w._version, w.device, dtype, tiled) for w in convw)
        cache = getattr(self, "_packed_cache", None)
        if cache is None or cache[0] != key:
            cache = (key, tuple(pack_conv_weight(w, dtype, tiled) for w in convw))
            self._packed_cache = cache
        return cache[1]

    def _packed_o_proj(self):
        """o_proj's weight in hydra_linear_fwd's fragment order, rebuilt only
        when the weight changes (tensor version counter) or moves."""
        w = self.o_proj.weight
        key = (w.data_ptr(), w._version, w.device, w.dtype)
        cache = getattr(self, "_packed_o_cache", None)
        if cache is None or cache[0] != key:
            cache = (key, pack_linear_weight(w))
            self._packed_o_cache = cache
        return cache[1]

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        """Legacy checkpoint migration (attention.py:333-383): q_conv1/q_conv2/
        k_conv1/k_conv2 -> q_conv.conv1/... and separate q/k/v(/v_shift)_down
        projections concatenated into qkv_proj."""
        has_q = hasattr(self, "q_conv")
        has_k = hasattr(self, "k_conv")
        for suffix in ("weight", "bias"):
            for old, new, has in (("q_conv1", "q_conv.conv1", has_q), ("q_conv2", "q_conv.conv2", has_q),
                                  ("k_conv1", "k_conv.conv1", has_k), ("k_conv2", "k_conv.conv2", has_k)):
                ok, nk = prefix + f"{old}.{suffix}", prefix + f"{new}.{suffix}"
                if ok not in state_dict:
                    continue
                if has and nk not in state_dict:
                    state_dict[nk] = state_dict.pop(ok)
                else:
                    state_dict.pop(ok, None)
        qk, kk, vk, vsk = (prefix + n for n in ("q_down.weight", "k_down.weight", "v_down.weight",
                                                "v_shift_down.weight"))
        fused = prefix + "qkv_proj.weight"
        if qk in state_dict and fused not in state_dict:
            parts = [state_dict.pop(qk), state_dict.pop(kk), state_dict.pop(vk)]
            if self.use_value_shift and vsk in state_dict:
                parts.append(state_dict.pop(vsk))
            state_dict[fused] = torch.cat(parts, dim=0)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)
