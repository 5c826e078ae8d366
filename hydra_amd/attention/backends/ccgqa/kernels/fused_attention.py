"""ccgqa_attention_fused (hydra/attention/backends/ccgqa/kernels/fused_attention.py:826-840)
on the gfx950 attention kernel: q [B,H,N,D], k/v [B,Hkv,N,D] -> out [B,H,N,D],
scale 1/sqrt(D), optional causal mask.  Forward only."""
from __future__ import annotations

import torch

from ....._autograd import track
from ..ops import attention_forward


def ccgqa_attention_fused(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          is_causal: bool = False, use_fused_backward: bool = True) -> torch.Tensor:
    """Public API of the fused CCGQA attention (fused_attention.py:826-840)."""
    with torch.no_grad():
        out, _ = attention_forward(q.detach(), k.detach(), v.detach(), causal=bool(is_causal))
    return track(out, q, k, v)


class CCGQAAttentionFused:
    """Name kept for callers of fused_attention.py:638; forward only."""

    @staticmethod
    def apply(q, k, v, is_causal=False, use_fused_backward=True):
        return ccgqa_attention_fused(q, k, v, is_causal, use_fused_backward)
