"""ccgqa_attention_fused (hydra/attention/backends/ccgqa/kernels/fused_attention.py:826-840)
on the gfx950 attention kernels: q [B,H,N,D], k/v [B,Hkv,N,D] -> out [B,H,N,D],
scale 1/sqrt(D), optional causal mask.  CCGQAAttentionFused is an autograd
Function like the reference's (:638-823): the forward keeps q, k, v, out and
the fp32 log-sum-exp, the backward runs the HIP split-K backward (dK/dV and
dQ launches, no atomics)."""
from __future__ import annotations

import torch

from ..ops import attention_backward, attention_forward


class CCGQAAttentionFused(torch.autograd.Function):
    """fused_attention.py:638-823.  `use_fused_backward` is accepted for the
    reference's signature; both of its settings run the HIP backward here
    (the reference's False branch recomputes the same gradients with torch
    matmuls, :791-821)."""

    @staticmethod
    def forward(ctx, q, k, v, is_causal=False, use_fused_backward=True):
        want = any(ctx.needs_input_grad[:3])
        out, lse = attention_forward(q, k, v, causal=bool(is_causal), want_lse=want)
        if want:
            ctx.save_for_backward(q, k, v, out, lse)
        ctx.is_causal = bool(is_causal)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = attention_backward(q, k, v, out, lse, grad_out, causal=ctx.is_causal)
        return dq, dk, dv, None, None


class MaskedAttentionFunction(torch.autograd.Function):
    """Attention with a padding mask: the SDPA call of CCGQAAttention.forward
    with its combined causal / padding attn_mask (attention.py:268-299),
    which the reference trains through autograd.  (q, k, v, key_mask [B,S],
    mask_mode, causal) -> out; the backward runs hydra_attn_bwd with the
    same mask."""

    @staticmethod
    def forward(ctx, q, k, v, key_mask, mask_mode, causal):
        want = any(ctx.needs_input_grad[:3])
        out, lse = attention_forward(q, k, v, causal=bool(causal), key_mask=key_mask,
                                     mask_mode=int(mask_mode), want_lse=want)
        if want:
            ctx.save_for_backward(q, k, v, out, lse, key_mask)
        ctx.causal, ctx.mask_mode = bool(causal), int(mask_mode)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, lse, key_mask = ctx.saved_tensors
        dq, dk, dv = attention_backward(q, k, v, out, lse, grad_out, causal=ctx.causal,
                                        key_mask=key_mask, mask_mode=ctx.mask_mode)
        return dq, dk, dv, None, None, None


def ccgqa_attention_fused(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          is_causal: bool = False, use_fused_backward: bool = True) -> torch.Tensor:
    """Public API of the fused CCGQA attention (fused_attention.py:826-840)."""
    return CCGQAAttentionFused.apply(q, k, v, is_causal, use_fused_backward)
