"""compute_token_losses_from_hidden (hydra/training/loop.py:28-89): per-token
cross-entropy losses from the final hidden states without keeping the full
logits, for loss-driven MoR routing and loss-aware MoD supervision."""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _lib
from ..kernels.fused_ops import _ce_rows


@torch.no_grad()
def compute_token_losses_from_hidden(hidden: torch.Tensor, weight: torch.Tensor,
                                     targets: torch.Tensor, ignore_index: int = -100,
                                     token_chunk_size: int = 2048,
                                     vocab_chunk_size: int = 4096) -> torch.Tensor:
    """[B, L] fp32 losses logsumexp(h W^T) - (h W^T)[t] in fp32, 0 at ignored
    positions.  Token chunks of `token_chunk_size` rows; each chunk's fp32
    logits go through hydra_ce_rows (the reference's vocab chunking,
    `vocab_chunk_size`, only bounds its temporary and is accepted for the
    signature).  Out-of-range targets: like the reference (:54-70), the whole
    target vector is clamped into [0, V) -- ignore_index entries included --
    and validity is recomputed afterwards."""
    _lib.require_gpu("compute_token_losses_from_hidden", hidden, weight, targets)
    B, L, D = hidden.shape
    V = weight.shape[0]
    N = B * L
    h = hidden.reshape(N, D)
    t = targets.reshape(N).to(torch.int64).clone()
    valid = t != ignore_index
    vt = t[valid]
    if vt.numel() > 0 and bool(((vt < 0) | (vt >= V)).any()):
        t.clamp_(min=0, max=V - 1)
    wf = weight.float()
    losses = torch.empty(N, dtype=torch.float32, device=hidden.device)
    for t0 in range(0, N, token_chunk_size):
        logits = F.linear(h[t0:t0 + token_chunk_size].float(), wf).contiguous()
        losses[t0:t0 + token_chunk_size] = _ce_rows(logits, t[t0:t0 + token_chunk_size], ignore_index)
    return losses.view(B, L)
