"""Mixture-of-Depths router and wrappers on gfx950
(hydra/routing/mixture_of_depths.py:92-301, model/framework/blocks.py:73-355).

The router's score GEMV stays on torch; the top-k select, the mask, the
ascending index list, the row gather and the scatters run in the HIP
kernels of libhydra_amd.so.  Gather and scatter are differentiable (their
backward runs the same kernels), so the wrappers train like the reference's.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .base import BaseRouter
from .ops import (gather_by_indices, mod_topk, router_k, scatter_replace,
                  weighted_residual_scatter)


def _aux_terms(scores: torch.Tensor, capacity_ratio: float) -> torch.Tensor:
    """capacity + collapse terms of the MoD load-balancing loss
    (mixture_of_depths.py:194-212; blocks.py:172-180)."""
    probs = torch.sigmoid(scores.clamp(-10.0, 10.0))
    capacity_loss = (probs.mean() - capacity_ratio).pow(2)
    expected_var = capacity_ratio * (1 - capacity_ratio) * 0.5
    collapse_loss = torch.exp(-probs.var() / max(expected_var, 0.01) * 5.0)
    return capacity_loss + 0.5 * collapse_loss


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

    @classmethod
    def from_config(cls, config) -> "MoDRouter":
        """mixture_of_depths.py:141-156 (any object with the MoDConfig fields)."""
        return cls(dim=config.dim, capacity_ratio=config.capacity_ratio,
                   aux_loss_weight=config.aux_loss_weight, jitter_noise=config.jitter_noise,
                   max_seq_len=config.max_seq_len)

    def select(self, x: torch.Tensor):
        """(scores [B,L], k, indices desc [B,k], indices ascending [B,k], mask [B,L])."""
        B, L, _ = x.shape
        k = router_k(L, self.capacity_ratio)
        scores = self.forward_logits(x)
        desc, srt, mask = mod_topk(scores.detach(), k, mask_dtype=x.dtype)
        if self.training and self.aux_loss_weight > 0:
            self._aux_loss = self.aux_loss_weight * _aux_terms(scores, self.capacity_ratio)
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
        x_sel = gather_by_indices(x, desc, distinct=True)
        y = self.block(x_sel, **kwargs)
        out = x.clone().to(y.dtype)
        return scatter_replace(out, y, desc)

    def get_aux_loss(self) -> torch.Tensor:
        return self.router.get_aux_loss()


class MoDMLPWrapper(nn.Module):
    """MoDMLPWrapper (blocks.py:73-355): Mixture-of-Depths on the MLP sublayer.

    Modes as in the reference: before routing is enabled (set_global_step past
    warmup_steps and, with enable_loss_threshold, the loss EMA below it) the
    dense mlp(x) with the router's aux loss; static_routing_mode computes
    every token and blends mlp(x) * p + x * (1 - p); otherwise hard top-k
    routing -- `_forward_hard` in eval, `_forward_hard_with_ste` in training
    (a zero-valued term that keeps the router's probabilities in the graph).
    forward_residual(h, x) fuses the caller's `h + wrapper(x)` (blocks.py:603)
    into the scatter on the hard path."""

    def __init__(self, mlp: nn.Module, dim: int, capacity_ratio: float = 0.5,
                 aux_loss_weight: float = 0.01, warmup_steps: int = 100,
                 force_enable_step: Optional[int] = None, max_seq_len: int = 2048,
                 enable_loss_threshold: Optional[float] = None, loss_aware_weight: float = 0.0,
                 static_routing_mode: bool = False):
        super().__init__()
        self.mlp = mlp
        self.capacity_ratio = capacity_ratio
        self.aux_loss_weight = aux_loss_weight
        self.warmup_steps = warmup_steps
        self.force_enable_step = (int(force_enable_step) if (force_enable_step is not None
                                                             and int(force_enable_step) > 0) else None)
        self.max_seq_len = max_seq_len
        self.loss_aware_weight = float(loss_aware_weight)
        self.static_routing_mode = static_routing_mode
        self.enable_loss_threshold = (float(enable_loss_threshold) if (enable_loss_threshold is not None
                                                                       and enable_loss_threshold > 0) else None)
        self._loss_unlocked = self.enable_loss_threshold is None
        self.register_buffer("_global_step", torch.zeros((), dtype=torch.int64), persistent=False)
        self.register_buffer("_zero_scalar", torch.tensor(0.0), persistent=False)
        self.register_buffer("_one_scalar", torch.tensor(1.0), persistent=False)
        self.register_buffer("_zero_int64", torch.zeros((), dtype=torch.int64), persistent=False)
        self.mod_router = MoDRouter(dim=dim, capacity_ratio=capacity_ratio,
                                    aux_loss_weight=aux_loss_weight, max_seq_len=max_seq_len)
        self._aux_loss = self._zero_scalar
        self._last_probs_mean_t = self._zero_scalar
        self._last_probs_std_t = self._zero_scalar
        self._routing_mode = "soft"
        self._tokens_processed = 0
        self._tokens_total = 0
        self._last_scores = None

    # -- schedule (blocks.py:136-161)
    def set_global_step(self, step: int) -> None:
        self._global_step.fill_(step)
        if self.force_enable_step is not None and step >= self.force_enable_step:
            self._loss_unlocked = True
        self._mod_enabled = (step >= self.warmup_steps) and self._loss_unlocked

    def update_loss_ema(self, loss_ema: float) -> None:
        if self._loss_unlocked:
            return
        if self.enable_loss_threshold is None:
            self._loss_unlocked = True
            return
        try:
            loss_val = float(loss_ema)
        except Exception:
            return
        if loss_val < self.enable_loss_threshold:
            self._loss_unlocked = True

    def _note_probs(self, scores: torch.Tensor) -> torch.Tensor:
        self._last_scores = scores
        probs = torch.sigmoid(scores.clamp(-10.0, 10.0))
        self._last_probs_mean_t = probs.mean().detach()
        self._last_probs_std_t = probs.std().detach()
        return probs

    def _dense_aux(self, scores: torch.Tensor) -> None:
        if self.training and self.aux_loss_weight > 0:
            self._aux_loss = self.aux_loss_weight * _aux_terms(scores, self.capacity_ratio)
        else:
            self._aux_loss = self._zero_scalar

    # -- forward paths
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.static_routing_mode:
            return self._forward_static(x)
        if not getattr(self, "_mod_enabled", False):
            self._routing_mode = "disabled"
            self._tokens_total = self._tokens_processed = x.shape[1]
            scores = self.mod_router.forward_logits(x)
            self._note_probs(scores)
            self._dense_aux(scores)
            return self.mlp(x)
        if not self.training:
            return self._forward_hard(x)
        return self._forward_hard_with_ste(x)

    def _forward_static(self, x: torch.Tensor) -> torch.Tensor:
        """blocks.py:190-241: every token through the MLP, blended by p."""
        self._routing_mode = "static"
        self._tokens_total = self._tokens_processed = x.shape[1]
        scores = self.mod_router.forward_logits(x)
        probs = self._note_probs(scores)
        self._dense_aux(scores)
        p = probs.unsqueeze(-1)
        return self.mlp(x) * p + x * (1 - p)

    def _route(self, x: torch.Tensor):
        scores, k, _, srt, _ = self.mod_router.select(x)
        self._last_indices = srt  # ascending selection of this call (diagnostics)
        probs = self._note_probs(scores)
        self._routing_mode = "hard"
        self._tokens_total, self._tokens_processed = x.shape[1], k
        if self.aux_loss_weight > 0:
            self._aux_loss = self.mod_router.get_aux_loss()
        return srt, probs

    def _forward_hard(self, x: torch.Tensor) -> torch.Tensor:
        """blocks.py:243-269: zeros except the selected rows, which hold
        mlp(x[selected]) (indices ascending)."""
        srt, _ = self._route(x)
        y = self.mlp(gather_by_indices(x, srt, distinct=True))
        out = torch.zeros_like(x, dtype=y.dtype)
        return scatter_replace(out, y.to(out.dtype), srt)

    def _forward_hard_with_ste(self, x: torch.Tensor) -> torch.Tensor:
        """blocks.py:271-300: the hard path plus a zero-valued term that keeps
        the selected tokens' router probabilities in the autograd graph."""
        srt, probs = self._route(x)
        y = self.mlp(gather_by_indices(x, srt, distinct=True))
        out = torch.zeros(x.shape, dtype=y.dtype, device=x.device)
        out = scatter_replace(out, y, srt)
        sel = torch.gather(probs, 1, srt)
        return out + (sel.sum() - sel.sum().detach()) * 0.0

    def forward_residual(self, h: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """h + forward(x), with the add fused into the scatter on the hard
        eval path (h is updated in place and returned there)."""
        if (self.static_routing_mode or not getattr(self, "_mod_enabled", False)
                or self.training):
            return h + self.forward(x)
        srt, _ = self._route(x)
        y = self.mlp(gather_by_indices(x, srt, distinct=True))
        return weighted_residual_scatter(h, y, srt)

    # -- losses and stats (blocks.py:302-355)
    def get_aux_loss(self) -> torch.Tensor:
        return self._aux_loss

    def compute_loss_aware_loss(self, token_losses: torch.Tensor) -> torch.Tensor:
        """blocks.py:305-335: BCE of the router scores against the top-k
        hardest tokens (lowest index wins ties, via the HIP top-k)."""
        if self.loss_aware_weight <= 0 or self._last_scores is None:
            return self._zero_scalar
        B, L = token_losses.shape
        k = int(max(1, min(L, int(L * float(self.capacity_ratio)))))
        valid_mask = torch.isfinite(token_losses)
        if not valid_mask.any():
            return self._zero_scalar
        with torch.no_grad():
            _, _, teacher = mod_topk(token_losses.float(), k, want_desc=False, want_sorted=False,
                                     mask_dtype=torch.float32)
            pos_weight = torch.tensor(float(max(1.0, (L - k) / max(1, k))),
                                      device=token_losses.device, dtype=torch.float32)
        per_tok = F.binary_cross_entropy_with_logits(self._last_scores.float().clamp(-10.0, 10.0),
                                                     teacher, pos_weight=pos_weight, reduction="none")
        loss = (per_tok * valid_mask.float()).sum() / valid_mask.float().sum().clamp_min(1.0)
        return loss * self.loss_aware_weight

    def get_routing_stats(self) -> dict:
        ratio = self._tokens_processed / max(1, self._tokens_total)
        return {
            "probs_mean": float(self._last_probs_mean_t.item()),
            "probs_std": float(self._last_probs_std_t.item()),
            "target_capacity": self.capacity_ratio,
            "tokens_processed": self._tokens_processed,
            "tokens_total": self._tokens_total,
            "compute_ratio": ratio,
            "compute_savings_pct": (1.0 - ratio) * 100.0,
            "routing_mode": self._routing_mode,
            "global_step": int(self._global_step),
            "warmup_steps": self.warmup_steps,
            "force_enable_step": self.force_enable_step,
            "enable_loss_threshold": self.enable_loss_threshold,
            "loss_unlocked": bool(self._loss_unlocked),
        }
