"""Training path of CCGQAAttention on gfx950: an autograd Function for the
q/k/v preparation (attention.py:205-266 and kernels/fused_conv.py:39-62,
which the reference trains through torch autograd).

forward:  hydra_ccgqa_prep_fwd (the inference kernel), keeping only qkv, the
          conv weights and the temperature.
backward: 1. the conv outputs y2 recomputed by the same kernel with the
             convs alone;
          2. hydra_ccgqa_prep_bwd: RoPE transpose, F.normalize backward
             (temperature gradient as per-token partials), QK-mean and
             value-shift backward -> grad(y2), the QK-mean and v parts of
             grad(qkv);
          3. the two k=3 causal convs as GEMMs over causal_im2col columns
             (hipBLASLt): conv2 -- dW2 = dY2^T im2col(y1),
             dy1 = col2im(dY2 W2r); conv1 (grouped, batched over groups) --
             dW1 = dY1^T im2col(q0), grad(q0) += col2im(dY1 W1r); y1 itself
             is recomputed as im2col(q0) W1r^T, rounded to the working dtype
             as the forward kernel rounds it.  Any conv kernel size (the
             taps of the im2col columns follow the weights).
"""
from __future__ import annotations

import torch

from ...._lib import CCGQA_CONVS, CCGQA_QK_NORM, CCGQA_W_TILED
from .ops import (causal_col2im, causal_im2col, ccgqa_prep, ccgqa_prep_backward,
                  tiled_weights_ok)


def _conv_pair_backward(x0: torch.Tensor, dy2: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                        groups: int, dx0: torch.Tensor):
    """Backward of y2 = conv2(conv1(x0)) (OptimizedConvSequence: conv1 with
    `groups`, conv2 dense, both k=3 causal) for x0 [B,S,C] and dy2 [B,S,C]
    (any row strides).  Adds grad(x0) into dx0 [B,S,C] and returns
    (dW1, dW2) in the weights' layouts [C, C/groups, 3] and [C, C, 3]."""
    B, S, C = x0.shape
    N, cg = B * S, C // groups
    ks = w1.shape[-1]  # conv taps
    dt = x0.dtype
    w1d, w2d = w1.detach().to(dt), w2.detach().to(dt)
    # Wr[g][o][t*cg + c] = W[g*cg + o, c, t]
    w1r = w1d.view(groups, cg, cg, ks).permute(0, 1, 3, 2).reshape(groups, cg, ks * cg).contiguous()
    w2r = w2d.permute(0, 2, 1).reshape(C, ks * C).contiguous()
    x0s = causal_im2col(x0, groups, ks)                            # [G, N, ks*cg]
    y1 = torch.bmm(x0s, w1r.transpose(1, 2).contiguous())         # [G, N, cg]
    y1 = y1.permute(1, 0, 2).reshape(B, S, C)
    y1s = causal_im2col(y1, 1, ks)[0]                              # [N, ks*C]
    dy2f = dy2.reshape(N, C)
    dw2 = (dy2f.t().contiguous() @ y1s).view(C, ks, C).permute(0, 2, 1)
    dy1 = torch.empty((B, S, C), dtype=dt, device=x0.device)
    causal_col2im((dy2f @ w2r).view(1, N, ks * C), dy1, taps=ks)
    dy1g = dy1.view(N, groups, cg).permute(1, 0, 2).contiguous()  # [G, N, cg]
    dw1 = torch.bmm(dy1g.transpose(1, 2).contiguous(), x0s)       # [G, cg, ks*cg]
    dw1 = dw1.view(groups, cg, ks, cg).permute(0, 1, 3, 2).reshape(C, cg, ks)
    causal_col2im(torch.bmm(dy1g, w1r), dx0, accumulate=True, taps=ks)
    return dw1.to(w1.dtype), dw2.to(w2.dtype)


class CCGQAPrepFunction(torch.autograd.Function):
    """(qkv, wq1, wq2, wk1, wk2, temperature, cos, sin, n_heads, n_kv_heads,
    head_dim, flags) -> (q [B,Hq,S,hd], k, v [B,Hkv,S,hd]); conv weights in
    Conv1d layout (None without convs), temperature None without QK-norm."""

    @staticmethod
    def forward(ctx, qkv, wq1, wq2, wk1, wk2, temperature, cos, sin, n_heads, n_kv_heads,
                head_dim, flags):
        convs = bool(flags & CCGQA_CONVS)
        ks = wq1.shape[-1] if convs else 3
        tiled = convs and ks == 3 and tiled_weights_ok(n_heads, n_kv_heads, head_dim, qkv.dtype)
        fl = flags | (CCGQA_W_TILED if tiled else 0)
        q, k, v = ccgqa_prep(qkv, n_heads, n_kv_heads, head_dim, fl, wq1, wq2, wk1, wk2,
                             temperature=temperature, cos=cos, sin=sin, conv_ks=ks)
        ctx.save_for_backward(qkv, wq1, wq2, wk1, wk2, temperature)
        ctx.rope = (cos, sin)
        ctx.meta = (n_heads, n_kv_heads, head_dim, flags, tiled)
        return q, k, v

    @staticmethod
    def backward(ctx, gq, gk, gv):
        qkv, wq1, wq2, wk1, wk2, temp = ctx.saved_tensors
        Hq, Hkv, hd, flags, tiled = ctx.meta
        cos, sin = ctx.rope
        B, S, _ = qkv.shape
        L, K = Hq * hd, Hkv * hd
        z = lambda h: torch.zeros((B, h, S, hd), dtype=qkv.dtype, device=qkv.device)
        gq = z(Hq) if gq is None else gq
        gk = z(Hkv) if gk is None else gk
        gv = z(Hkv) if gv is None else gv
        convs = bool(flags & CCGQA_CONVS)
        y2q = y2k = None
        if convs:
            fl = CCGQA_CONVS | (CCGQA_W_TILED if tiled else 0)
            y2q, y2k, _ = ccgqa_prep(qkv, Hq, Hkv, hd, fl, wq1, wq2, wk1, wk2, conv_ks=wq1.shape[-1])
        dy, dqkv, dtemp_tok = ccgqa_prep_backward(qkv, Hq, Hkv, hd, flags, gq, gk, gv, y2q, y2k,
                                                  temperature=temp, cos=cos, sin=sin)
        dw = [None] * 4
        if convs:
            dw[0], dw[1] = _conv_pair_backward(qkv[..., :L], dy[..., :L], wq1, wq2, Hq, dqkv[..., :L])
            dw[2], dw[3] = _conv_pair_backward(qkv[..., L:L + K], dy[..., L:], wk1, wk2, Hkv,
                                               dqkv[..., L:L + K])
        dtemp = None
        if temp is not None and (flags & CCGQA_QK_NORM) and ctx.needs_input_grad[5]:
            dtemp = dtemp_tok.sum().reshape(temp.shape).to(temp.dtype)
        return (dqkv, *dw, dtemp, None, None, None, None, None, None)


def ccgqa_prep_train(qkv, n_heads, n_kv_heads, head_dim, flags, wq1=None, wq2=None, wk1=None,
                     wk2=None, temperature=None, cos=None, sin=None):
    """ccgqa_prep with a backward (q, k, v in [B,H,S,hd]; no V_TRANSPOSED)."""
    return CCGQAPrepFunction.apply(qkv, wq1, wq2, wk1, wk2, temperature, cos, sin, n_heads,
                                   n_kv_heads, head_dim, flags)
