"""MovingAverageBaseline (hydra/routing/loss_tracker.py:37-140): the EMA of
per-token losses HydraModel keeps for loss-driven MoR routing.  Kept for the
model's state_dict layout (its four persistent buffers) and for the
advantage signal of the routing losses; nothing here runs on the forward
path."""
from __future__ import annotations

import torch
import torch.nn as nn


class MovingAverageBaseline(nn.Module):
    def __init__(self, decay: float = 0.99, warmup_steps: int = 1000) -> None:
        super().__init__()
        self.decay = decay
        self.warmup_steps = warmup_steps
        self.register_buffer("_ema", torch.tensor(0.0), persistent=True)
        self.register_buffer("_ema_var", torch.tensor(1.0), persistent=True)
        self.register_buffer("_step", torch.tensor(0, dtype=torch.long), persistent=True)
        self.register_buffer("_initialized", torch.tensor(False), persistent=True)

    @property
    def baseline(self) -> float:
        return self._ema.item()

    @property
    def baseline_std(self) -> float:
        return max(0.01, self._ema_var.sqrt().item())

    @property
    def step(self) -> int:
        return self._step.item()

    @property
    def is_active(self) -> bool:
        """Past warmup (loss_tracker.py:81-84)."""
        return self._step.item() >= self.warmup_steps

    @torch.no_grad()
    def update(self, token_losses: torch.Tensor) -> None:
        """EMA of the batch mean and (unbiased) variance (:86-108)."""
        flat = token_losses.detach().flatten()
        mean, var = flat.mean(), flat.var()
        if not bool(self._initialized):
            self._ema.copy_(mean)
            self._ema_var.copy_(var)
            self._initialized.fill_(True)
        else:
            self._ema.mul_(self.decay).add_(mean * (1 - self.decay))
            self._ema_var.mul_(self.decay).add_(var * (1 - self.decay))
        self._step.add_(1)

    def compute_advantage(self, token_losses: torch.Tensor) -> torch.Tensor:
        """tanh((loss - ema) / max(0.01, sqrt(ema_var))), zero during warmup
        (:110-133)."""
        if not self.is_active:
            return torch.zeros_like(token_losses)
        std = max(0.01, self._ema_var.sqrt().item())
        return torch.tanh((token_losses - self._ema) / std)
