"""HydraModel on gfx950 (hydra/model/framework/model.py:166-809): token
embedding (hydra_embedding_fwd), the HydraMoRBlock stack (MoD on the MLP of
the middle blocks), the final RMSNorm and the (tied) LM head.  Same
constructor, submodule names and state_dict keys as the reference, so its
checkpoints load (hydra_amd.training.load_module_from_checkpoint)."""
from __future__ import annotations

import math
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from ... import _lib
from ..._autograd import track
from ...layers import RMSNorm
from ...routing.loss_tracker import MovingAverageBaseline
from .blocks import HydraMoRBlock


def embedding_lookup(table: torch.Tensor, ids: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """_safe_embedding_lookup (model.py:51-73): table[clamp(ids, 0, V-1)] *
    scale, one launch (the reference's out-of-range warning needs a host
    synchronisation and is not kept)."""
    _lib.require_gpu("embedding_lookup", table, ids)
    V, dim = table.shape
    idx = ids.reshape(-1).to(torch.int64).contiguous()
    t = table if table.stride(-1) == 1 else table.contiguous()
    out = torch.empty((idx.numel(), dim), dtype=table.dtype, device=table.device)
    with torch.cuda.device(table.device):
        _lib.call("hydra_embedding_fwd", idx.data_ptr(), idx.numel(), t.data_ptr(), V, dim,
                  t.stride(0), float(scale), out.data_ptr(), dim, _lib.dtype_code(table),
                  _lib.stream(table))
    return track(out.view(*ids.shape, dim), table)


class HydraModel(nn.Module):
    """model.py:166-809 (MoE layers, gradient checkpointing and the
    diagnostics accessors are not part of this build)."""

    def __init__(self, vocab_size: int = 50257, dim: int = 1536, n_mor_blocks: int = 4,
                 recursions_per_block: int = 6, n_heads: int = 24, n_kv_heads: int = 4,
                 compression_factor: int = 4, mlp_ratio: float = 2.67, max_seq_len: int = 8192,
                 mod_capacity: float = 0.5, aux_loss_weight: float = None, adaptive: bool = True,
                 tie_weights: bool = True, hybrid_attention: bool = True,
                 mod_loss_aware_weight: float = 0.0, dim_ref: int = 768, depth_alpha: float = 0.0,
                 depth_scale_max: float = 2.0, attention_backend: str = "ccgqa",
                 mor_min_depth: int = 0, static_routing_mode: bool = False,
                 moe_enabled: bool = False, **kwargs):
        super().__init__()
        if moe_enabled:
            raise NotImplementedError("HydraModel: MoE layers are not part of this build")
        self.dim = dim
        self.vocab_size = vocab_size
        self.n_mor_blocks = n_mor_blocks
        self.recursions_per_block = recursions_per_block
        self.effective_layers = n_mor_blocks * recursions_per_block
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.compression_factor = compression_factor
        self.mlp_ratio = mlp_ratio
        self.max_seq_len = max_seq_len
        self.mod_capacity = mod_capacity
        self.mod_loss_aware_weight = float(mod_loss_aware_weight)
        self.adaptive = adaptive
        self.hybrid_attention = hybrid_attention
        self.attention_backend = attention_backend.lower() if attention_backend else "ccgqa"
        self.dim_ref, self.depth_alpha, self.depth_scale_max = dim_ref, depth_alpha, depth_scale_max
        self.moe_enabled = False
        self.mor_min_depth = mor_min_depth
        self.static_routing_mode = static_routing_mode
        if aux_loss_weight is None:  # model.py:267-270
            depth_scale = max(1.0, self.effective_layers / 32)
            dim_scale = max(1.0, (dim / 768) ** 0.5)
            aux_loss_weight = 0.5 * depth_scale * dim_scale
        self.aux_loss_weight = aux_loss_weight
        self.register_buffer("_global_step", torch.zeros((), dtype=torch.int64), persistent=False)
        self.register_buffer("_zero_scalar", torch.tensor(0.0), persistent=False)

        self.tok_emb = nn.Embedding(vocab_size, dim)
        self._attention_pattern = ["ccqa"] * n_mor_blocks
        self.layers = nn.ModuleList()
        for i in range(n_mor_blocks):
            use_mod_mlp = 0 < i < n_mor_blocks - 1  # model.py:283
            self.layers.append(HydraMoRBlock(
                dim=dim, n_heads=n_heads, n_kv_heads=n_kv_heads,
                compression_factor=compression_factor, mlp_ratio=mlp_ratio,
                max_seq_len=max_seq_len, max_recursions=recursions_per_block, adaptive=adaptive,
                layer_idx=i, total_layers=n_mor_blocks, attention_type="ccqa",
                mod_mlp_capacity=mod_capacity if use_mod_mlp else None,
                mod_mlp_aux_weight=self.aux_loss_weight if use_mod_mlp else 0.0,
                mod_mlp_warmup=kwargs.get("mod_mlp_warmup", 100),
                mod_force_enable_step=kwargs.get("mod_force_enable_step", None),
                mod_enable_loss_threshold=kwargs.get("mod_enable_loss_threshold", None),
                mod_loss_aware_weight=self.mod_loss_aware_weight,
                mor_warmup=kwargs.get("mor_warmup", 1000), dim_ref=dim_ref,
                depth_alpha=depth_alpha, depth_scale_max=depth_scale_max,
                mor_min_depth=mor_min_depth, static_routing_mode=static_routing_mode))
        self.moe_layers = nn.ModuleList()
        self._moe_placement = ()
        self.norm = RMSNorm(dim)
        self.output = nn.Linear(dim, vocab_size, bias=False)
        self.loss_baseline = MovingAverageBaseline(decay=0.99, warmup_steps=1000)
        self._init_weights()
        if tie_weights:
            self.output.weight = self.tok_emb.weight

    def _init_weights(self) -> None:
        """model.py:346-373: N(0, 0.02) for Linear / Embedding / Conv1d
        weights, router biases kept, o_proj and down scaled by
        1/sqrt(2 * effective_layers)."""
        residual_scale = 1.0 / math.sqrt(2 * self.effective_layers)
        for name, module in self.named_modules():
            if isinstance(module, nn.Linear):
                nn.init.normal_(module.weight, mean=0.0, std=0.02)
                if module.bias is not None and "router" not in name:
                    nn.init.zeros_(module.bias)
                if "o_proj" in name or "down" in name:
                    module.weight.data *= residual_scale
            elif isinstance(module, (nn.Embedding, nn.Conv1d)):
                nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def resize_rope_cache(self, new_max_seq_len: int) -> None:
        for layer in self.layers:
            attn = layer.attention
            if attn.use_rope and attn.cos_cached.shape[2] < new_max_seq_len:
                device = attn.cos_cached.device
                attn._init_rope(new_max_seq_len)
                attn.cos_cached = attn.cos_cached.to(device)
                attn.sin_cached = attn.sin_cached.to(device)
        self.max_seq_len = new_max_seq_len

    def _embed(self, x: torch.Tensor) -> torch.Tensor:
        return embedding_lookup(self.tok_emb.weight, x, scale=math.sqrt(self.dim))

    def forward_hidden(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Post-norm hidden states (model.py:504-540)."""
        h = self._embed(x)
        for layer in self.layers:
            h = layer(h)
        return self.norm(h)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None,
                return_losses: bool = False) -> Union[torch.Tensor, Tuple[torch.Tensor, dict]]:
        """Logits [B, S, vocab] (model.py:408-502)."""
        if not return_losses:
            return F.linear(self.forward_hidden(x), self.output.weight)
        h = self._embed(x)
        results = []
        for layer in self.layers:
            h, losses = layer.forward_with_losses(h)
            results.append(losses)
        logits = F.linear(self.norm(h), self.output.weight)
        aux = [r["aux_loss"] for r in results if "aux_loss" in r]
        ponder = [r["ponder_loss"] for r in results if "ponder_loss" in r]
        z = self._zero_scalar
        return logits, {"aux_loss": sum(aux) if aux else z, "ponder_loss": sum(ponder) if ponder else z,
                        "moe_aux_loss": z, "moe_teacher_loss": z}

    def set_global_step(self, step: int) -> None:
        """model.py:695-705."""
        self._global_step.fill_(step)
        self._cached_global_step = step
        self._mor_adaptive_cached = step >= getattr(self, "_mor_enable_step", 0)
        for layer in self.layers:
            layer.set_global_step(step)

    def set_mor_curriculum(self, enable_step: int, rampup_steps: int = 1000) -> None:
        self._mor_enable_step = enable_step
        self._mor_rampup_steps = rampup_steps
        for layer in self.layers:
            layer.set_mor_enable_step(enable_step, rampup_steps)

    def trigger_mor_early(self, current_step: int, rampup_steps: int = 1000) -> None:
        """model.py:722-728."""
        self.set_mor_curriculum(current_step, rampup_steps)

    def update_mod_loss_ema(self, loss_ema: float) -> None:
        for layer in self.layers:
            if layer.mod_mlp_wrapper is not None:
                layer.mod_mlp_wrapper.update_loss_ema(loss_ema)
