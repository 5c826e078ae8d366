"""Thin tensor-level wrappers over the CCGQA entry points of the C ABI
(hydra_ccgqa_prep_fwd, hydra_attn_fwd, hydra_linear_fwd).  Shapes and dtypes are checked
here; strides, pointers and the current stream go to the library."""
from __future__ import annotations

import ctypes

from typing import Optional

import torch
import torch.nn.functional as F

from ...._lib import (CCGQA_CONVS, CCGQA_QK_MEAN, CCGQA_QK_NORM, CCGQA_ROPE,
                      CCGQA_V_TRANSPOSED, CCGQA_VALUE_SHIFT, CCGQA_W_TILED, MASK_KEY_PADDING, MASK_NONE,
                      MASK_REFERENCE_SDPA)
from .... import _lib


def prep_flags(use_convs: bool, use_qk_mean: bool, use_value_shift: bool,
               use_qk_norm: bool, use_rope: bool) -> int:
    return ((CCGQA_CONVS if use_convs else 0) | (CCGQA_QK_MEAN if use_qk_mean else 0)
            | (CCGQA_VALUE_SHIFT if use_value_shift else 0)
            | (CCGQA_QK_NORM if use_qk_norm else 0) | (CCGQA_ROPE if use_rope else 0))


def pack_conv_weight(w: torch.Tensor, dtype: torch.dtype, tiled: bool = False) -> torch.Tensor:
    """Conv1d weight [out, in/groups, k] -> the tap-major [k, out, in/groups]
    layout the prep kernel reads, or with `tiled` its MFMA-fragment order
    [k, out/32, in/16, 2, 32, 8] (CCGQA_W_TILED): element (t, o/32, i/16,
    (i/8)%2, o%32, i%8), so one 32x16 operand block is contiguous."""
    t = w.detach().to(dtype).permute(2, 0, 1)
    if not tiled:
        return t.contiguous()
    k, O, I = t.shape
    return t.reshape(k, O // 32, 32, I // 16, 2, 8).permute(0, 1, 3, 4, 2, 5).contiguous()


def tiled_weights_ok(n_heads: int, n_kv_heads: int, head_dim: int, dtype: torch.dtype) -> bool:
    """Whether the prep kernel takes its MFMA path for this head layout and
    dtype, i.e. accepts CCGQA_W_TILED weights."""
    if dtype not in _lib._DTYPE_CODE:
        return False
    return _lib.query("hydra_ccgqa_prep_tiled_ok", n_heads, n_kv_heads, head_dim,
                      _lib._DTYPE_CODE[dtype]) == 1


def ccgqa_prep(qkv: torch.Tensor, n_heads: int, n_kv_heads: int, head_dim: int, flags: int,
               wq1=None, wq2=None, wk1=None, wk2=None, temperature=None, cos=None, sin=None,
               packed: bool = False, conv_ks: int = 3):
    """q [B,Hq,S,hd], k/v [B,Hkv,S,hd] from the fused projection qkv [B,S,L+2K]
    (CCGQAAttention.forward, attention.py:205-266).  Conv weights are in
    PyTorch Conv1d layout, or already packed (pack_conv_weight, tiled when
    CCGQA_W_TILED is in flags) when packed=True.  With
    CCGQA_V_TRANSPOSED in flags, v is returned as a [B,Hkv,S,hd] view of a
    [B,Hkv,hd,S] buffer (the layout the attention kernel stages directly)."""
    _lib.require_gpu("ccgqa_prep", qkv, wq1, wq2, wk1, wk2, temperature, cos, sin)
    B, S, W = qkv.shape
    L, K = n_heads * head_dim, n_kv_heads * head_dim
    if W != L + 2 * K:
        raise ValueError(f"ccgqa_prep: qkv width {W} != L + 2K = {L + 2 * K}")
    if qkv.stride(-1) != 1 or (B > 1 and qkv.stride(0) != S * qkv.stride(1)):
        qkv = qkv.contiguous()
    dt = qkv.dtype
    if flags & CCGQA_CONVS:
        ws = (wq1, wq2, wk1, wk2)
        tiled = bool(flags & CCGQA_W_TILED)
        if packed:
            ws = tuple(w.to(dt).contiguous() for w in ws)
        else:
            ws = tuple(pack_conv_weight(w, dt, tiled) for w in ws)
        ks = conv_ks
        exp = [(ks, L, head_dim), (ks, L, L), (ks, K, head_dim), (ks, K, K)]
        if tiled:
            exp = [(ks, o // 32, i // 16, 2, 32, 8) for _, o, i in exp]
        for w, e in zip(ws, exp):
            if tuple(w.shape) != e:
                raise ValueError(f"ccgqa_prep: packed conv weight shape {tuple(w.shape)} != {e}")
        wq1, wq2, wk1, wk2 = ws
    else:
        wq1 = wq2 = wk1 = wk2 = None
    temp = None if temperature is None else temperature.detach().to(dt).contiguous()
    if flags & CCGQA_ROPE:
        if cos.dim() == 4:
            cos, sin = cos[0, 0], sin[0, 0]
        if cos.shape[0] < S:
            raise ValueError(f"ccgqa_prep: RoPE cache covers {cos.shape[0]} positions < S={S}")
        cos = cos[:S].float().contiguous()
        sin = sin[:S].float().contiguous()
    q = torch.empty((B, n_heads, S, head_dim), dtype=dt, device=qkv.device)
    k = torch.empty((B, n_kv_heads, S, head_dim), dtype=dt, device=qkv.device)
    vt = bool(flags & CCGQA_V_TRANSPOSED)
    v = torch.empty((B, n_kv_heads, head_dim, S) if vt else (B, n_kv_heads, S, head_dim),
                    dtype=dt, device=qkv.device)
    with torch.cuda.device(qkv.device):
        _lib.call("hydra_ccgqa_prep_fwd", qkv.data_ptr(), qkv.stride(1), _lib.ptr(wq1),
                  _lib.ptr(wq2), _lib.ptr(wk1), _lib.ptr(wk2), _lib.ptr(temp), _lib.ptr(cos),
                  _lib.ptr(sin), head_dim // 2 if cos is None else cos.stride(0),
                  q.data_ptr(), k.data_ptr(), v.data_ptr(), B, S, n_heads, n_kv_heads,
                  head_dim, conv_ks, flags, _lib.dtype_code(qkv), _lib.stream(qkv))
    return q, k, (v.transpose(2, 3) if vt else v)


def attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool,
                      scale: Optional[float] = None, key_mask: Optional[torch.Tensor] = None,
                      mask_mode: int = MASK_NONE, out: Optional[torch.Tensor] = None,
                      want_lse: bool = False, score_bound: Optional[float] = None,
                      bound_temperature: Optional[torch.Tensor] = None):
    """Softmax attention over [B,H,S,hd] q and [B,Hkv,S,hd] k/v.  `out` may be
    any [B,Hq,S,hd]-indexed view (e.g. a [B,S,Hq,hd] buffer transposed).
    score_bound: optional beta >= max |q.k| (before the scale); with one the
    bf16 kernel takes a fixed reference max instead of a running row max
    (see qk_norm_score_bound).  bound_temperature: a one-element bf16/fp32
    tensor on the device whose qk_norm_score_bound the kernel takes itself
    at launch (no host sync; graph replays follow later values).  Returns
    (out, lse or None)."""
    _lib.require_gpu("attention_forward", q, k, v, key_mask, out)
    B, Hq, S, hd = q.shape
    Hkv = k.shape[1]
    if k.shape != (B, Hkv, S, hd) or v.shape != (B, Hkv, S, hd):
        raise ValueError(f"attention_forward: k/v shapes {tuple(k.shape)}, {tuple(v.shape)} "
                         f"do not match q {tuple(q.shape)}")
    if Hq % Hkv != 0:
        raise ValueError("attention_forward: n_heads must be a multiple of n_kv_heads")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("attention_forward: q, k, v must share a dtype")
    q, k = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k))
    if v.stride(-1) != 1 and v.stride(-2) != 1:
        v = v.contiguous()
    if out is None:
        out = torch.empty((B, Hq, S, hd), dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.stride(-1) != 1:
        raise ValueError("attention_forward: out must be a [B,Hq,S,hd] view with unit last stride")
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device) if want_lse else None
    km = None
    if mask_mode != MASK_NONE:
        if key_mask is None or key_mask.shape != (B, S):
            raise ValueError(f"attention_forward: key mask must be [B,S] = [{B},{S}]")
        km = (key_mask != 0).to(torch.uint8).contiguous()
    sc = float(hd ** -0.5) if scale is None else float(scale)
    bt = None
    if bound_temperature is not None:
        bt = bound_temperature.detach()
        if bt.dtype not in (torch.bfloat16, torch.float32):
            bt = bt.float()
        bt = bt.reshape(-1)[:1].contiguous()
        _lib.require_gpu("attention_forward", bt)
    with torch.cuda.device(q.device):
        st = (_lib.strides(q), _lib.strides(k), _lib.strides(v), _lib.strides(out))
        need = ctypes.c_int64(0)
        _lib.call("hydra_attn_fwd_workspace", B, Hq, Hkv, S, hd, *st, 1 if causal else 0, mask_mode,
                  _lib.dtype_code(q), ctypes.byref(need))
        ws = _lib.scratch(need.value, q) if need.value else None
        _lib.call("hydra_attn_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                  _lib.ptr(lse), _lib.ptr(km), mask_mode, B, Hq, Hkv, S, hd, *st,
                  1 if causal else 0, sc, float(score_bound or 0.0), _lib.ptr(bt),
                  0 if bt is None else _lib.dtype_code(bt), _lib.dtype_code(q), _lib.ptr(ws),
                  need.value, _lib.stream(q))
    return out, lse


def attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                       lse: torch.Tensor, grad_out: torch.Tensor, *, causal: bool,
                       scale: Optional[float] = None, key_mask: Optional[torch.Tensor] = None,
                       mask_mode: int = MASK_NONE):
    """Gradients (dq, dk, dv) of attention_forward's output, from the forward's
    inputs, its output and its fp32 log-sum-exp (want_lse=True): the split-K
    backward of CCGQAAttentionFused (fused_attention.py:706-823, kernels
    :113-338 and :432-635).  dk and dv sum the Hq/Hkv query heads that share
    a K/V head.  key_mask / mask_mode: those of the forward call (the
    backward of the padding-mask SDPA call, attention.py:268-299)."""
    _lib.require_gpu("attention_backward", q, k, v, out, lse, grad_out)
    B, Hq, S, hd = q.shape
    Hkv = k.shape[1]
    if k.shape != (B, Hkv, S, hd) or v.shape != (B, Hkv, S, hd) or out.shape != q.shape \
            or grad_out.shape != q.shape:
        raise ValueError(f"attention_backward: shapes q {tuple(q.shape)}, k {tuple(k.shape)}, "
                         f"v {tuple(v.shape)}, out {tuple(out.shape)}, grad {tuple(grad_out.shape)}")
    if Hq % Hkv != 0:
        raise ValueError("attention_backward: n_heads must be a multiple of n_kv_heads")
    if not (q.dtype == k.dtype == v.dtype == out.dtype):
        raise ValueError("attention_backward: q, k, v and out must share a dtype")
    if lse.shape != (B, Hq, S) or lse.dtype != torch.float32:
        raise ValueError("attention_backward: lse must be fp32 [B, Hq, S]")
    q, k, v, out = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v, out))
    grad_out = grad_out.to(q.dtype)
    grad_out = grad_out if grad_out.stride(-1) == 1 else grad_out.contiguous()
    lse = lse.contiguous()
    dq, dk, dv = torch.empty_like(q, memory_format=torch.contiguous_format), \
        torch.empty_like(k, memory_format=torch.contiguous_format), \
        torch.empty_like(v, memory_format=torch.contiguous_format)
    sc = float(hd ** -0.5) if scale is None else float(scale)
    km = None
    if mask_mode != MASK_NONE:
        if key_mask is None or key_mask.shape != (B, S):
            raise ValueError(f"attention_backward: key mask must be [B,S] = [{B},{S}]")
        _lib.require_gpu("attention_backward", key_mask)
        km = (key_mask != 0).to(torch.uint8).contiguous()
    with torch.cuda.device(q.device):
        st = (_lib.strides(q), _lib.strides(k), _lib.strides(v), _lib.strides(out),
              _lib.strides(grad_out), _lib.strides(dq), _lib.strides(dk), _lib.strides(dv))
        need = ctypes.c_int64(0)
        _lib.call("hydra_attn_bwd_workspace", B, Hq, Hkv, S, hd, *st, mask_mode, 1 if causal else 0,
                  _lib.dtype_code(q), ctypes.byref(need))
        ws = _lib.scratch(need.value, q)
        _lib.call("hydra_attn_bwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                  grad_out.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                  B, Hq, Hkv, S, hd, *st, _lib.ptr(km), mask_mode, 1 if causal else 0, sc,
                  _lib.dtype_code(q), _lib.ptr(ws), need.value, _lib.stream(q))
    return dq, dk, dv


def linear_weight_ok(weight: torch.Tensor) -> bool:
    """Whether hydra_linear_fwd takes this [N, K] weight (bf16, K in
    {64, 128, 256}, N % 64 == 0)."""
    N, K = weight.shape
    return weight.dtype == torch.bfloat16 and K in (64, 128, 256) and N % 64 == 0


def pack_linear_weight(weight: torch.Tensor) -> torch.Tensor:
    """[N, K] -> the MFMA-fragment order hydra_linear_fwd reads with
    HYDRA_LINEAR_W_TILED: [N/32, K/16, 2, 32, 8], element [j, s, h, n, e] =
    weight[32 j + n, 16 s + 8 h + e]."""
    N, K = weight.shape
    return (weight.detach().reshape(N // 32, 32, K // 16, 2, 8).permute(0, 2, 3, 1, 4)
            .contiguous())


def output_projection(x: torch.Tensor, weight: torch.Tensor,
                      packed: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F.linear(x, weight) without bias: CCGQAAttention's o_proj
    (attention.py:329-331).  bf16 rows of width 64, 128 or 256 with
    weight.shape[0] % 64 == 0 go to hydra_linear_fwd (with `packed`, the
    weight already in pack_linear_weight's order; else it is packed here);
    other shapes (and a recorded autograd graph, which the kernel has no
    backward for) stay on the library GEMM, as in the reference."""
    N, K = weight.shape
    if (torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad)) or \
            x.dtype != torch.bfloat16 or not linear_weight_ok(weight) or x.shape[-1] != K:
        return F.linear(x, weight)
    _lib.require_gpu("output_projection", x, weight, packed)
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w = pack_linear_weight(weight) if packed is None else packed
    y = torch.empty(*x.shape[:-1], N, device=x.device, dtype=x.dtype)
    rc = _lib.call_status("hydra_linear_fwd", x2.data_ptr(), x2.stride(0), w.data_ptr(), K, y.data_ptr(), N,
                          x2.shape[0], N, K, _lib.LINEAR_W_TILED, _lib.BF16, _lib.stream(x))
    if rc == _lib.ERR_UNSUPPORTED:  # unaligned rows
        return F.linear(x, weight)
    _lib.check(rc, "hydra_linear_fwd")
    return y


def qk_norm_score_bound(temperature: float) -> float:
    """Bound on |q.k| after CCGQAAttention's QK L2-norm (attention.py:260-262):
    q has unit norm and k the norm |temperature|, RoPE is a rotation, and the
    bf16 roundings of the norm, the normalised vector, the temperature product
    and RoPE move a norm by less than 1%; 3% covers it."""
    return 1.03 * abs(float(temperature))


def conv_sequence(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, groups1: int,
                  groups2: int) -> torch.Tensor:
    """Standalone OptimizedConvSequence forward ([B,N,C] -> [B,N,C]) through
    the prep kernel's conv stage: x is laid out as the q block of a qkv
    buffer whose k block is zero, with every other prep feature off."""
    if groups2 != 1:
        raise NotImplementedError("conv_sequence: the HIP conv stage implements a dense conv2 (groups2 == 1)")
    _lib.require_gpu("conv_sequence", x, w1, w2)
    B, N, C = x.shape
    hd = C // groups1
    ks = w1.shape[-1]
    qkv = torch.zeros((B, N, C + 2 * hd), dtype=x.dtype, device=x.device)
    qkv[..., :C] = x
    zk = torch.zeros((hd, hd, ks), dtype=x.dtype, device=x.device)
    q, _, _ = ccgqa_prep(qkv, groups1, 1, hd, CCGQA_CONVS, w1, w2, zk, zk, conv_ks=ks)
    return q.transpose(1, 2).reshape(B, N, C)


__all__ = ["prep_flags", "pack_conv_weight", "ccgqa_prep", "attention_forward", "conv_sequence",
           "qk_norm_score_bound", "MASK_NONE", "MASK_KEY_PADDING", "MASK_REFERENCE_SDPA"]


def causal_im2col(x: torch.Tensor, groups: int, taps: int = 3) -> torch.Tensor:
    """[B,S,G*cg] (unit channel stride, any row stride) -> [G, B*S, taps*cg]:
    row b*S+s of group g holds x[b, s+t-(taps-1), g*cg:(g+1)*cg] for taps
    t = 0..taps-1 (zero before the row start), the operand of the causal
    conv as a GEMM (hydra_causal_im2col)."""
    _lib.require_gpu("causal_im2col", x)
    B, S, C = x.shape
    if C % groups != 0:
        raise ValueError(f"causal_im2col: {C} channels not divisible by {groups} groups")
    if x.stride(-1) != 1 or (B > 1 and x.stride(0) != S * x.stride(1)):
        x = x.contiguous()
    cg = C // groups
    out = torch.empty((groups, B * S, taps * cg), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("hydra_causal_im2col", x.data_ptr(), x.stride(1), out.data_ptr(), B, S, groups, cg,
                  taps, _lib.dtype_code(x), _lib.stream(x))
    return out


def causal_col2im(cols: torch.Tensor, out: torch.Tensor, accumulate: bool = False,
                  taps: int = 3) -> torch.Tensor:
    """The transpose of causal_im2col: cols [G, B*S, taps*cg] summed over
    taps into out [B,S,G*cg] (unit channel stride; added to its contents
    with `accumulate`).  Returns out."""
    _lib.require_gpu("causal_col2im", cols, out)
    B, S, C = out.shape
    G = cols.shape[0]
    if C % G != 0 or cols.shape != (G, B * S, taps * (C // G)) or cols.dtype != out.dtype:
        raise ValueError(f"causal_col2im: cols {tuple(cols.shape)} do not match out {tuple(out.shape)}")
    if out.stride(-1) != 1 or (B > 1 and out.stride(0) != S * out.stride(1)):
        raise ValueError("causal_col2im: out needs unit channel stride and uniform row stride")
    cols = cols.contiguous()
    with torch.cuda.device(out.device):
        _lib.call("hydra_causal_col2im", cols.data_ptr(), out.data_ptr(), out.stride(1), B, S, G,
                  C // G, taps, 1 if accumulate else 0, _lib.dtype_code(out), _lib.stream(out))
    return out


def ccgqa_prep_backward(qkv: torch.Tensor, n_heads: int, n_kv_heads: int, head_dim: int, flags: int,
                        dq: torch.Tensor, dk: torch.Tensor, dv: torch.Tensor, y2q=None, y2k=None,
                        temperature=None, cos=None, sin=None):
    """Pointwise backward of ccgqa_prep (hydra_ccgqa_prep_bwd): returns
    (dy [B,S,L+K] or None, dqkv [B,S,L+2K], dtemp_tok fp32 [B*S] or None).
    dy is the gradient of the conv outputs (CCGQA_CONVS); dqkv holds the
    QK-mean and v parts of grad(qkv) (and the direct q0/k0 part without
    convs)."""
    _lib.require_gpu("ccgqa_prep_backward", qkv, dq, dk, dv, y2q, y2k, temperature, cos, sin)
    B, S, W = qkv.shape
    L, K = n_heads * head_dim, n_kv_heads * head_dim
    if W != L + 2 * K:
        raise ValueError(f"ccgqa_prep_backward: qkv width {W} != L + 2K = {L + 2 * K}")
    if qkv.stride(-1) != 1 or (B > 1 and qkv.stride(0) != S * qkv.stride(1)):
        qkv = qkv.contiguous()
    dt = qkv.dtype
    dq, dk, dv = (t.to(dt).contiguous() for t in (dq, dk, dv))
    convs = bool(flags & CCGQA_CONVS)
    if convs:
        y2q, y2k = y2q.to(dt).contiguous(), y2k.to(dt).contiguous()
    dy = torch.empty((B, S, L + K), dtype=dt, device=qkv.device) if convs else None
    dqkv = torch.empty((B, S, W), dtype=dt, device=qkv.device)
    norm = bool(flags & CCGQA_QK_NORM)
    dtemp = torch.empty(B * S, dtype=torch.float32, device=qkv.device) if norm else None
    temp = None if temperature is None else temperature.detach().to(dt).contiguous()
    if flags & CCGQA_ROPE:
        if cos.dim() == 4:
            cos, sin = cos[0, 0], sin[0, 0]
        cos = cos[:S].float().contiguous()
        sin = sin[:S].float().contiguous()
    with torch.cuda.device(qkv.device):
        _lib.call("hydra_ccgqa_prep_bwd", qkv.data_ptr(), qkv.stride(1), _lib.ptr(y2q), _lib.ptr(y2k),
                  _lib.ptr(temp), _lib.ptr(cos), _lib.ptr(sin),
                  head_dim // 2 if cos is None else cos.stride(0), dq.data_ptr(), dk.data_ptr(),
                  dv.data_ptr(), _lib.ptr(dy), dqkv.data_ptr(), dqkv.stride(1), _lib.ptr(dtemp), B, S,
                  n_heads, n_kv_heads, head_dim, flags & ~CCGQA_W_TILED, _lib.dtype_code(qkv),
                  _lib.stream(qkv))
    return dy, dqkv, dtemp
