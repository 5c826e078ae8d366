"""Mixture-of-Recursions on gfx950 (hydra/routing/mixture_of_recursions.py).

MoRRouter: the router's Linear(dim, 1) stays a torch GEMV; the depth
mapping (tanh clamp, sigmoid, rounding to a recursion index) runs in
hydra_mor_route.  MoRExecutor: each recursion's pre-norm input
(current + recursion bias + recursion embedding, normalised) is one
hydra_residual_norm_fwd launch, and the masked state update plus the exit
accumulation one hydra_mor_update launch; the MLP between them is the
caller's module (SwiGLU GEMMs, or the MoD wrapper).  Forward only: the
straight-through gradient path of the reference is not built, and a
backward through these ops raises."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _lib
from .._autograd import track
from ..layers.common import residual_norm
from .base import BaseRouter

__all__ = ["MoRConfig", "MoRRouter", "MoRExecutor", "MoROutput", "dim_to_depth_scale",
           "compute_layer_target_prob"]


@dataclass(frozen=True)
class MoRConfig:
    """mixture_of_recursions.py:65-105 (same fields, defaults and checks)."""
    dim: int
    n_recursions: int = 5
    ponder_loss_weight: float = 0.01
    router_jitter: float = 0.0
    warmup_steps: int = 2500
    layer_idx: int = 0
    total_layers: int = 1
    dim_ref: int = 768
    depth_alpha: float = 0.0
    depth_scale_max: float = 2.0
    advantage_loss_scale: float = 0.1
    min_depth: int = 0
    static_routing_mode: bool = False

    def __post_init__(self) -> None:
        if self.dim <= 0:
            raise ValueError(f"dim must be positive, got {self.dim}")
        if self.n_recursions < 1:
            raise ValueError(f"n_recursions must be >= 1, got {self.n_recursions}")
        if self.ponder_loss_weight < 0:
            raise ValueError(f"ponder_loss_weight must be >= 0, got {self.ponder_loss_weight}")


@dataclass
class MoROutput:
    hidden_states: torch.Tensor
    ponder_loss: torch.Tensor
    depths: torch.Tensor
    router_probs: torch.Tensor
    router_logits: torch.Tensor


def dim_to_depth_scale(dim: int, dim_ref: int = 768, depth_alpha: float = 0.0,
                       scale_max: float = 2.0) -> float:
    """mixture_of_recursions.py:130-155."""
    if depth_alpha <= 0.0 or dim <= dim_ref:
        return 1.0
    return min((dim / dim_ref) ** depth_alpha, scale_max)


def compute_layer_target_prob(layer_idx: int, total_layers: int, depth_scale: float = 1.0) -> float:
    """mixture_of_recursions.py:158-187: 0.2 for the first layer rising
    linearly to 0.5 for the last, shifted deeper by depth_scale > 1."""
    base = 0.2 + 0.3 * (layer_idx / max(1, total_layers - 1))
    if depth_scale > 1.0:
        return float(1.0 - (1.0 - base) / depth_scale)
    return float(base)


def mor_route(logits: torch.Tensor, n_recursions: int, min_depth: int = 0):
    """(depths int64, probs, clamped logits) from raw router logits [B, L]
    (hydra_mor_route; mixture_of_recursions.py:259-288)."""
    _lib.require_gpu("mor_route", logits)
    lg = logits.contiguous()
    probs = torch.empty_like(lg)
    lout = torch.empty_like(lg)
    depths = torch.empty(lg.shape, dtype=torch.int64, device=lg.device)
    with torch.cuda.device(lg.device):
        _lib.call("hydra_mor_route", lg.data_ptr(), lg.numel(), probs.data_ptr(), lout.data_ptr(),
                  depths.data_ptr(), int(n_recursions), int(min_depth), _lib.dtype_code(lg),
                  _lib.stream(lg))
    return depths, probs, lout


def mor_update(current: torch.Tensor, delta: torch.Tensor, output: torch.Tensor,
               depths: torch.Tensor, recursion: int) -> None:
    """In place: current += delta * (depth >= i); output += current * (depth == i)
    (hydra_mor_update; mixture_of_recursions.py:466-476)."""
    _lib.require_gpu("mor_update", current, delta, output, depths)
    dim = current.shape[-1]
    c2, o2 = current.view(-1, dim), output.view(-1, dim)
    d2 = delta.to(current.dtype).reshape(-1, dim)
    if d2.stride(-1) != 1:
        d2 = d2.contiguous()
    dep = depths.reshape(-1).to(torch.int64).contiguous()
    with torch.cuda.device(current.device):
        _lib.call("hydra_mor_update", c2.data_ptr(), c2.stride(0), d2.data_ptr(), d2.stride(0),
                  o2.data_ptr(), o2.stride(0), dep.data_ptr(), c2.shape[0], dim, int(recursion),
                  _lib.dtype_code(current), _lib.stream(current))


class MoRRouter(BaseRouter):
    """mixture_of_recursions.py:194-351: per-token recursion depth from a
    learned Linear(dim, 1), bias initialised to the layer's target
    probability."""

    def __init__(self, config: MoRConfig) -> None:
        super().__init__(config.dim, config.router_jitter)
        self.config = config
        self._depth_scale = dim_to_depth_scale(config.dim, config.dim_ref, config.depth_alpha,
                                               config.depth_scale_max)
        self._target_prob = compute_layer_target_prob(config.layer_idx, config.total_layers,
                                                      self._depth_scale)
        self._init_bias(self._target_prob)
        nn.init.normal_(self.router.weight, mean=0.0, std=0.02)
        self._warmup_steps = config.warmup_steps
        self.register_buffer("_global_step", torch.zeros((), dtype=torch.int64), persistent=False)
        self.register_buffer("_zero_scalar", torch.tensor(0.0), persistent=False)
        self._cached_global_step = 0

    def set_global_step(self, step: int) -> None:
        self._global_step.fill_(step)
        self._cached_global_step = step

    @property
    def warmup_scale(self) -> float:
        return min(1.0, self._cached_global_step / max(1, self._warmup_steps))

    def forward(self, x: torch.Tensor, return_continuous: bool = False
                ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(depths [B, L] int64 in [min_depth, R-1], probs, clamped logits)."""
        logits = self.forward_logits(x)
        depths, probs, lout = mor_route(logits.detach(), self.config.n_recursions,
                                        self.config.min_depth)
        return depths, track(probs, logits), track(lout, logits)

    def compute_ponder_loss(self, depths: torch.Tensor, probs: torch.Tensor, logits: torch.Tensor,
                            token_losses: Optional[torch.Tensor] = None,
                            baseline=None) -> torch.Tensor:
        """mixture_of_recursions.py:290-351 (small [B, L] reductions, torch)."""
        n_rec = self.config.n_recursions
        depth_continuous = probs * (n_rec - 1)
        ponder_cost = depth_continuous.mean() / float(max(1, n_rec - 1))
        collapse_loss = torch.exp(-probs.var() * 10.0)
        logit_var_loss = F.relu(0.5 - logits.var())
        if token_losses is not None and baseline is not None:
            advantage = baseline.compute_advantage(token_losses)
            advantage_loss = -(advantage * depth_continuous).mean() * float(self.config.advantage_loss_scale)
        else:
            advantage_loss = self._zero_scalar
        ponder = 0.0005 * ponder_cost + 0.01 * collapse_loss + 0.1 * logit_var_loss + advantage_loss
        return torch.clamp(self.warmup_scale * ponder, max=5.0)


class MoRExecutor(nn.Module):
    """mixture_of_recursions.py:358-558: R passes of `mlp` sharing weights;
    token t's state moves only while i <= depth[t], and the output takes the
    state at i == depth[t].  Static mode blends every recursion's state by
    normalised Gaussian depth weights."""

    def __init__(self, config: MoRConfig) -> None:
        super().__init__()
        self.config = config
        self.recursion_bias = nn.Parameter(torch.zeros(config.n_recursions, 1, 1, config.dim) * 0.02)
        self.recursion_embed = nn.Embedding(config.n_recursions, config.dim)
        nn.init.normal_(self.recursion_embed.weight, std=0.02)
        self.register_buffer("_recursion_indices", torch.arange(config.n_recursions, dtype=torch.long),
                             persistent=False)
        self._recursion_tokens_processed: list = []

    def _rec_vectors(self, i: int):
        return self.recursion_bias[i].reshape(-1), self.recursion_embed.weight[i]

    def _pre(self, current: torch.Tensor, i: int, norm: Optional[nn.Module]) -> torch.Tensor:
        """norm(current + recursion_bias[i] + recursion_embed[i]) in one
        launch when `norm` is one of this package's norms."""
        b1, b2 = self._rec_vectors(i)
        mode = getattr(norm, "_hydra_norm_mode", None)
        if mode is not None:
            _, y = residual_norm(current, b1=b1, b2=b2, weight=norm.weight, eps=norm.eps, norm=mode)
            return y
        h, _ = residual_norm(current, b1=b1, b2=b2, norm=_lib.NORM_NONE)
        return norm(h) if norm is not None else h

    def forward(self, x: torch.Tensor, depths: torch.Tensor, probs: torch.Tensor, mlp: nn.Module,
                norm: Optional[nn.Module] = None) -> torch.Tensor:
        if self.config.static_routing_mode:
            return self._forward_static(x, probs, mlp, norm)
        n_rec = self.config.n_recursions
        with torch.no_grad():
            current = x.detach().clone()
            output = torch.zeros_like(current)
            if self.training:
                self._recursion_tokens_processed = [(depths >= i).sum() for i in range(n_rec)]
            for i in range(n_rec):
                delta = mlp(self._pre(current, i, norm))
                mor_update(current, delta, output, depths, i)
        return track(output, x, probs, *self.parameters(), *mlp.parameters())

    def _forward_static(self, x: torch.Tensor, probs: torch.Tensor, mlp: nn.Module,
                        norm: Optional[nn.Module] = None) -> torch.Tensor:
        """mixture_of_recursions.py:480-549 (torch elementwise on the
        [R, B, L] weights; the MLP passes are the caller's)."""
        n_rec = self.config.n_recursions
        dc = probs * (n_rec - 1)
        idx = torch.arange(n_rec, device=x.device, dtype=x.dtype)
        w = torch.exp(-((dc.unsqueeze(0) - idx.view(-1, 1, 1)) ** 2))
        w = w / (w.sum(dim=0, keepdim=True) + 1e-8)
        output = torch.zeros_like(x)
        current = x
        for i in range(n_rec):
            current = current + mlp(self._pre(current, i, norm))
            output = output + w[i].unsqueeze(-1) * current
        return output

    def get_recursion_stats(self) -> dict:
        if not self._recursion_tokens_processed:
            return {}
        return {f"depth_{i}_tokens": t.item() for i, t in enumerate(self._recursion_tokens_processed)}
