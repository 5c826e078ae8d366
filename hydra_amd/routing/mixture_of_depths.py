"""Mixture-of-Depths router and wrappers on gfx950
(hydra/routing/mixture_of_depths.py:92-301, model/framework/blocks.py:73-300).

The router's score GEMV stays on torch; the top-k select, the mask, the
ascending index list, the row gather and the residual scatter run in the HIP
kernels of libhydra_amd.so.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .base import BaseRouter
from .ops import (gather_by_indices, mod_topk, router_k, scatter_replace,
                  weighted_residual_scatter)


class MoDRouter(BaseRouter):
    """mixture_of_depths.py:92-220."""

    def __init__(self, dim: int, capacity_ratio: float = 0.5, aux_loss_weight: float = 0.01,
                 jitter_noise: float = 0.0, max_seq_len: int = 2048):
        super().__init__(dim, jitter_noise)
        self.capacity_ratio = capacity_ratio
        self.aux_loss_weight = aux_loss_weight
        self.max_seq_len = max_seq_len
        self.static_k = max(1, int(max_seq_len * capacity_ratio))
        nn.init.normal_(self.router.weight, mean=0.0, std=0.02)
        self._init_bias(self.capacity_ratio)
        self.register_buffer("_aux_loss", torch.tensor(0.0))

    def _aux(self, scores: torch.Tensor) -> None:
        """Load-balancing loss (mixture_of_depths.py:194-212)."""
        probs = torch.sigmoid(scores.clamp(-10.0, 10.0))
        capacity_loss = (probs.mean() - self.capacity_ratio).pow(2)
        expected_var = self.capacity_ratio * (1 - self.capacity_ratio) * 0.5
        collapse_loss = torch.exp(-probs.var() / max(expected_var, 0.01) * 5.0)
        self._aux_loss = self.aux_loss_weight * (capacity_loss + 0.5 * collapse_loss)

    def select(self, x: torch.Tensor):
        """(scores [B,L], k, indices desc [B,k], indices ascending [B,k], mask [B,L])."""
        B, L, _ = x.shape
        k = router_k(L, self.capacity_ratio)
        scores = self.forward_logits(x)
        desc, srt, mask = mod_topk(scores.detach(), k, mask_dtype=x.dtype)
        if self.training and self.aux_loss_weight > 0:
            self._aux(scores)
        return scores, k, desc, srt, mask

    def forward(self, x: torch.Tensor, return_scores: bool = False
                ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
        scores, _, desc, _, mask = self.select(x)
        return mask, desc, (scores if return_scores else None)

    def get_aux_loss(self) -> torch.Tensor:
        return self._aux_loss


class MixtureOfDepthsBlock(nn.Module):
    """mixture_of_depths.py:223-301: selected tokens go through `block`, the
    others keep their input values."""

    def __init__(self, block: nn.Module, dim: int, capacity_ratio: float = 0.5,
                 aux_loss_weight: float = 0.01):
        super().__init__()
        self.block = block
        self.router = MoDRouter(dim=dim, capacity_ratio=capacity_ratio, aux_loss_weight=aux_loss_weight)

    def forward(self, x: torch.Tensor, **kwargs) -> torch.Tensor:
        B, L, D = x.shape
        _, k, desc, _, _ = self.router.select(x)
        if k == L:
            return self.block(x, **kwargs)
        x_sel = gather_by_indices(x, desc)
        y = self.block(x_sel, **kwargs)
        out = x.clone().to(y.dtype)
        return scatter_replace(out, y, desc)

    def get_aux_loss(self) -> torch.Tensor:
        return self.router.get_aux_loss()


class MoDMLPWrapper(nn.Module):
    """The hard-routing path of MoDMLPWrapper (blocks.py:73-269).

    forward(x) is `_forward_hard` once routing is enabled (set_global_step
    past warmup_steps) and the dense `mlp(x)` before that; forward_residual
    fuses the caller's residual add (`h + wrapper(x)`, blocks.py:603) into the
    scatter."""

    def __init__(self, mlp: nn.Module, dim: int, capacity_ratio: float = 0.5,
                 aux_loss_weight: float = 0.01, warmup_steps: int = 100,
                 max_seq_len: int = 2048):
        super().__init__()
        self.mlp = mlp
        self.capacity_ratio = capacity_ratio
        self.aux_loss_weight = aux_loss_weight
        self.warmup_steps = warmup_steps
        self.mod_router = MoDRouter(dim=dim, capacity_ratio=capacity_ratio,
                                    aux_loss_weight=aux_loss_weight, max_seq_len=max_seq_len)
        self._mod_enabled = False
        self._tokens_processed = 0
        self._tokens_total = 0

    def set_global_step(self, step: int) -> None:
        self._mod_enabled = step >= self.warmup_steps

    def _route(self, x):
        _, k, _, srt, _ = self.mod_router.select(x)
        self._tokens_total, self._tokens_processed = x.shape[1], k
        return srt

    def _forward_hard(self, x: torch.Tensor) -> torch.Tensor:
        """blocks.py:243-269: zeros except the selected rows, which hold
        mlp(x[selected]) (indices sorted ascending before the gather)."""
        srt = self._route(x)
        y = self.mlp(gather_by_indices(x, srt))
        out = torch.zeros_like(x, dtype=y.dtype)
        return scatter_replace(out, y, srt)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self._mod_enabled:
            return self.mlp(x)
        return self._forward_hard(x)

    def forward_residual(self, h: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """h + forward(x) with the add fused into the scatter (h is updated in
        place and returned)."""
        if not self._mod_enabled:
            return h.add_(self.mlp(x))
        srt = self._route(x)
        y = self.mlp(gather_by_indices(x, srt))
        return weighted_residual_scatter(h, y, srt)
