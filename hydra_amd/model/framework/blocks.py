"""HydraBlock and HydraMoRBlock on gfx950 (hydra/model/framework/blocks.py).

Same constructors, submodule names and state_dict keys as the reference.
In inference (no autograd recording) the residual adds are fused into the
following pre-norm (hydra_residual_norm_fwd) and the MLP's residual into its
down-projection GEMM; when autograd records, the blocks run their modules
one by one so every differentiable op keeps its backward."""
from __future__ import annotations

import os
from typing import Optional, Tuple

import torch
import torch.nn as nn

from ... import _lib
from ...attention.backends.ccgqa.attention import CCGQAAttention
from ...attention.factory import build_hybrid_attention_module
from ...layers import AdaRMSNorm, RMSNorm, SwiGLUMLPFused, residual_norm
from ...routing.mixture_of_depths import MoDMLPWrapper
from ...routing.mixture_of_recursions import (MoRConfig, MoRExecutor, MoRRouter,
                                               dim_to_depth_scale)

SwiGLUMLP = SwiGLUMLPFused


def _recording(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)


def _mlp_residual(mlp: nn.Module, h: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """h + mlp(y), the add in the GEMM epilogue for the SwiGLU MLP."""
    if isinstance(mlp, SwiGLUMLPFused):
        return mlp.forward_residual(h, y)
    return h + mlp(y)


class HydraBlock(nn.Module):
    """blocks.py:33-70: pre-norm block, h = x + attn(norm1(x));
    out = h + mlp(norm2(h)); hidden = int(dim * mlp_ratio) rounded up to a
    multiple of 256 (blocks.py:64-65)."""

    def __init__(self, dim: int, n_heads: int = 16, n_kv_heads: int = 4,
                 compression_factor: int = 4, mlp_ratio: float = 2.67, max_seq_len: int = 8192,
                 norm_eps: float = 1e-6, **attention_kwargs):
        super().__init__()
        self.attention = CCGQAAttention(dim=dim, n_heads=n_heads, n_kv_heads=n_kv_heads,
                                        compression_factor=compression_factor,
                                        max_seq_len=max_seq_len, **attention_kwargs)
        self.norm1 = RMSNorm(dim, eps=norm_eps)
        self.norm2 = RMSNorm(dim, eps=norm_eps)
        hidden_dim = int(dim * mlp_ratio)
        hidden_dim = ((hidden_dim + 255) // 256) * 256
        self.mlp = SwiGLUMLP(dim, hidden_dim)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        a = self.attention(self.norm1(x), mask=mask)
        if _recording(x, a, *self.norm2.parameters(), *self.mlp.parameters()):
            h = x + a
            return h + self.mlp(self.norm2(h))
        h, y = residual_norm(x, r=a, weight=self.norm2.weight, eps=self.norm2.eps,
                             norm=_lib.NORM_RMS, want_h=True)
        return _mlp_residual(self.mlp, h, y)


class HydraMoRBlock(nn.Module):
    """blocks.py:431-756: attention once, then up to `max_recursions` passes
    of the (optionally MoD-wrapped) MLP per token, depth chosen by the MoR
    router; AdaRMSNorm pre-norms (HYDRA_USE_ADA_RMSNORM, default on), a
    final RMSNorm, residual_scale 0.5 on the attention branch."""

    def __init__(self, dim: int, n_heads: int = 16, n_kv_heads: int = 4,
                 compression_factor: int = 4, mlp_ratio: float = 2.67, max_seq_len: int = 8192,
                 max_recursions: int = 6, adaptive: bool = True, halt_threshold: float = 0.9,
                 ponder_loss_weight: float = 0.01, layer_idx: int = 0, total_layers: int = 1,
                 attention_type: str = "lla3", dim_ref: int = 768, depth_alpha: float = 0.0,
                 depth_scale_max: float = 2.0, static_routing_mode: bool = False,
                 **attention_kwargs):
        super().__init__()
        self.max_recursions = max_recursions
        self.adaptive = adaptive
        self.layer_idx = layer_idx
        self.total_layers = total_layers
        self.dim = dim
        self.attention_type = attention_type
        self.static_routing_mode = static_routing_mode
        self._depth_scale = dim_to_depth_scale(dim, dim_ref, depth_alpha, depth_scale_max)

        mod_mlp_capacity = attention_kwargs.pop("mod_mlp_capacity", None)
        mod_mlp_aux_weight = attention_kwargs.pop("mod_mlp_aux_weight", 0.01)
        mod_mlp_warmup = attention_kwargs.pop("mod_mlp_warmup", 100)
        mod_force_enable_step = attention_kwargs.pop("mod_force_enable_step", None)
        mod_enable_loss_threshold = attention_kwargs.pop("mod_enable_loss_threshold", None)
        mod_loss_aware_weight = attention_kwargs.pop("mod_loss_aware_weight", 0.0)
        mor_warmup = attention_kwargs.pop("mor_warmup", 1000)
        self.use_mod_mlp = mod_mlp_capacity is not None and mod_mlp_capacity > 0

        # HydraModel passes "ccqa"; other names raise in the factory, as in
        # the reference (whose default "lla3" has no backend either).
        self.attention = build_hybrid_attention_module(
            attention_type, dim=dim,
            n_heads=n_heads, n_kv_heads=n_kv_heads, max_seq_len=max_seq_len,
            compression_factor=compression_factor, attention_kwargs=attention_kwargs)
        self.residual_scale = 0.5
        Norm = AdaRMSNorm if os.environ.get("HYDRA_USE_ADA_RMSNORM", "1") == "1" else RMSNorm
        self.norm1 = Norm(dim)
        hidden_dim = int(dim * mlp_ratio)
        hidden_dim = ((hidden_dim + 255) // 256) * 256
        self.mlp = SwiGLUMLP(dim, hidden_dim)
        self.norm2 = Norm(dim)
        if self.use_mod_mlp:
            self.mod_mlp_wrapper = MoDMLPWrapper(
                mlp=self.mlp, dim=dim, capacity_ratio=mod_mlp_capacity,
                aux_loss_weight=mod_mlp_aux_weight, warmup_steps=mod_mlp_warmup,
                force_enable_step=mod_force_enable_step, max_seq_len=max_seq_len,
                enable_loss_threshold=mod_enable_loss_threshold,
                loss_aware_weight=mod_loss_aware_weight, static_routing_mode=static_routing_mode)
        else:
            self.mod_mlp_wrapper = None
        self.block = None

        mor_min_depth = attention_kwargs.pop("mor_min_depth", 0)
        mor_config = MoRConfig(
            dim=dim, n_recursions=max_recursions, ponder_loss_weight=ponder_loss_weight,
            warmup_steps=mor_warmup, layer_idx=layer_idx, total_layers=total_layers,
            dim_ref=dim_ref, depth_alpha=depth_alpha, depth_scale_max=depth_scale_max,
            advantage_loss_scale=attention_kwargs.pop("mor_advantage_loss_scale", 0.1),
            min_depth=mor_min_depth, static_routing_mode=static_routing_mode)
        self.mor_router = MoRRouter(mor_config)
        self.mor_executor = MoRExecutor(mor_config)
        self._mor_config = mor_config
        self.ponder_loss_weight = ponder_loss_weight

        self.register_buffer("_global_step", torch.zeros((), dtype=torch.int64), persistent=False)
        self.register_buffer("_zero_scalar", torch.tensor(0.0), persistent=False)
        self.register_buffer("_one_scalar", torch.tensor(1.0), persistent=False)
        self.register_buffer("_zero_int64", torch.zeros((), dtype=torch.int64), persistent=False)
        self._warmup_steps = 2500
        self._mor_enable_step = 0
        self._mor_rampup_steps = 0
        self.final_norm = RMSNorm(dim)
        self._ponder_loss = self._zero_scalar
        self._last_target_depths: Optional[torch.Tensor] = None

    # -- pieces
    def _attn_residual(self, x: torch.Tensor) -> torch.Tensor:
        """x + residual_scale * attention(norm1(x)) (blocks.py:615-619),
        the scale and the add in one launch."""
        a = self.attention(self.norm1(x))
        if _recording(x, a):
            return x + self.residual_scale * a
        h, _ = residual_norm(x, r=a, alpha=self.residual_scale, norm=_lib.NORM_NONE)
        return h

    def _mlp(self) -> nn.Module:
        return self.mod_mlp_wrapper if self.mod_mlp_wrapper is not None else self.mlp

    def _forward_fixed(self, x: torch.Tensor) -> torch.Tensor:
        """blocks.py:601-612: every recursion for every token."""
        h = self._attn_residual(x)
        ex = self.mor_executor
        for i in range(self.max_recursions):
            y = ex._pre(h, i, self.norm2)
            mlp = self._mlp()
            if isinstance(mlp, SwiGLUMLPFused) and not _recording(h, y):
                h = mlp.forward_residual(h, y)
            else:
                h = h + mlp(y)
        return self.final_norm(h)

    def _forward_mor(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """blocks.py:614-633."""
        h = self._attn_residual(x)
        depths, probs, logits = self.mor_router(h)
        self._last_target_depths = depths.detach().float()
        self._last_router_probs_tensor = probs.detach()
        self._last_router_logits = logits
        self._last_depths = depths
        self._last_probs = probs
        output = self.mor_executor(h, depths, probs, self._mlp(), self.norm2)
        ponder_loss = self.mor_router.compute_ponder_loss(depths, probs, logits)
        if self.training:
            n_rec = self.max_recursions
            self._ponder_loss = ponder_loss.detach()
            self._last_avg_depth = (probs * (n_rec - 1)).mean().detach()
        return self.final_norm(output), ponder_loss

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """blocks.py:652-663: the MoR ramp blends the adaptive and fixed paths."""
        if self.adaptive:
            ramp = self.get_mor_rampup_scale()
            if ramp <= 0.0:
                return self._forward_fixed(x)
            out, _ = self._forward_mor(x)
            if ramp >= 1.0:
                return out
            return ramp * out + (1.0 - ramp) * self._forward_fixed(x)
        return self._forward_fixed(x)

    def forward_with_losses(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None):
        """blocks.py:665-697."""
        aux = self.mod_mlp_wrapper.get_aux_loss if self.mod_mlp_wrapper is not None else None
        if self.adaptive:
            ramp = self.get_mor_rampup_scale()
            if ramp > 0.0:
                out, ponder = self._forward_mor(x)
                ponder = ponder * ramp
                aux_loss = aux() if aux else self._zero_scalar
                if ramp < 1.0:
                    out = ramp * out + (1.0 - ramp) * self._forward_fixed(x)
                if self.training:
                    self._ponder_loss = ponder.detach()
                return out, {"ponder_loss": ponder, "aux_loss": aux_loss}
        out = self._forward_fixed(x)
        if self.training:
            self._ponder_loss = self._zero_scalar
        return out, {"ponder_loss": self._zero_scalar, "aux_loss": aux() if aux else self._zero_scalar}

    def get_ponder_loss(self) -> torch.Tensor:
        return self._ponder_loss

    # -- schedule (blocks.py:731-756)
    def set_global_step(self, step: int) -> None:
        self._global_step.fill_(step)
        self._cached_global_step = step
        self._mor_adaptive_cached = step >= self._mor_enable_step
        if step < self._mor_enable_step:
            self._mor_rampup_scale_cached = 0.0
        elif self._mor_rampup_steps <= 0:
            self._mor_rampup_scale_cached = 1.0
        else:
            raw = min(1.0, (step - self._mor_enable_step + 1) / self._mor_rampup_steps)
            self._mor_rampup_scale_cached = max(0.1, round(raw * 10) / 10)
        if self.mod_mlp_wrapper is not None:
            self.mod_mlp_wrapper.set_global_step(step)

    def set_mor_enable_step(self, enable_step: int, rampup_steps: int = 1000) -> None:
        self._mor_enable_step = enable_step
        self._mor_rampup_steps = rampup_steps

    def is_mor_adaptive_enabled(self) -> bool:
        return getattr(self, "_mor_adaptive_cached", False)

    def get_mor_rampup_scale(self) -> float:
        return getattr(self, "_mor_rampup_scale_cached", 1.0)

    def get_aux_loss(self) -> torch.Tensor:
        return self.mod_mlp_wrapper.get_aux_loss() if self.mod_mlp_wrapper is not None else self._zero_scalar
