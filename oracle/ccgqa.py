"""Oracle for the CCGQA attention forward
(hydra/attention/backends/ccgqa/attention.py:201-331 with
OptimizedConvSequence, kernels/fused_conv.py:39-62).

Functional form over an explicit parameter dict whose keys are the
CCGQAAttention state_dict keys (attention.py:114-147):
  qkv_proj.weight, o_proj.weight, q_conv.conv1.weight, q_conv.conv2.weight,
  k_conv.conv1.weight, k_conv.conv2.weight, key_temperature.

Test infrastructure only: see oracle/__init__.py.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import fused_ops


@dataclass
class CCGQAConfig:
    dim: int
    n_heads: int = 16
    n_kv_heads: int = 4
    compression_factor: int = 4
    max_seq_len: int = 8192
    use_rope: bool = True
    use_qk_norm: bool = True
    use_convs: bool = True
    use_qk_mean: bool = True
    use_value_shift: bool = True
    conv_kernel_size: int = 3
    output_scale: float = 1.0

    @property
    def latent_dim(self) -> int:  # attention.py:103
        return self.dim // self.compression_factor

    @property
    def head_dim(self) -> int:  # attention.py:104
        return self.latent_dim // self.n_heads

    @property
    def kv_dim(self) -> int:  # attention.py:105
        return self.n_kv_heads * self.head_dim

    @property
    def n_groups(self) -> int:  # attention.py:93
        return self.n_heads // self.n_kv_heads


def init_params(cfg: CCGQAConfig, generator: torch.Generator, std: float = 0.02,
                temperature: float | None = None, dtype=torch.float32) -> dict:
    """N(0, std) weights in the shapes of attention.py:114-147 (Conv1d weight
    [out, in/groups, k]); key_temperature defaults to sqrt(head_dim)
    (attention.py:147)."""
    L, K, hd, ks = cfg.latent_dim, cfg.kv_dim, cfg.head_dim, cfg.conv_kernel_size
    shapes = {
        "qkv_proj.weight": (L + 2 * K, cfg.dim),
        "o_proj.weight": (cfg.dim, L),
    }
    if cfg.use_convs:
        shapes.update({
            "q_conv.conv1.weight": (L, L // cfg.n_heads, ks),
            "q_conv.conv2.weight": (L, L, ks),
            "k_conv.conv1.weight": (K, K // cfg.n_kv_heads, ks),
            "k_conv.conv2.weight": (K, K, ks),
        })
    p = {n: (torch.randn(s, generator=generator) * std).to(dtype) for n, s in shapes.items()}
    t = math.sqrt(hd) if temperature is None else temperature
    p["key_temperature"] = torch.full((1,), float(t)).to(dtype)
    return p


def causal_conv_seq(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                    groups1: int) -> torch.Tensor:
    """OptimizedConvSequence.forward (fused_conv.py:39-62): [B,N,C] ->
    transpose, left-pad k-1, conv1 (groups1), left-pad k-1, conv2 (dense),
    transpose back."""
    pad = w1.shape[-1] - 1
    y = x.transpose(1, 2).contiguous()
    y = F.conv1d(F.pad(y, (pad, 0)), w1, groups=groups1)
    y = F.conv1d(F.pad(y, (pad, 0)), w2, groups=1)
    return y.transpose(1, 2).contiguous()


def prep(params: dict, qkv: torch.Tensor, cfg: CCGQAConfig, cos=None, sin=None):
    """attention.py:205-266: split, value shift, convs, QK-mean, QK-norm,
    RoPE.  Returns q [B,Hq,S,hd], k [B,Hkv,S,hd], v [B,Hkv,S,hd]."""
    B, S, _ = qkv.shape
    L, K, hd = cfg.latent_dim, cfg.kv_dim, cfg.head_dim
    q = qkv[..., :L]
    k = qkv[..., L:L + K]
    if cfg.use_value_shift:  # attention.py:211-220
        v_curr = qkv[..., L + K:L + K + K // 2]
        v_prev = qkv[..., L + K + K // 2:]
        half = K // 2
        v = torch.empty((B, S, K), dtype=qkv.dtype)
        v[..., :half] = v_curr
        v[..., half:] = 0
        v[:, 1:, half:] = v_prev[:, :-1, :]
    else:
        v = qkv[..., L + K:]
    q_pre, k_pre = q, k
    if cfg.use_convs:  # attention.py:228-231
        q = causal_conv_seq(q, params["q_conv.conv1.weight"], params["q_conv.conv2.weight"], cfg.n_heads)
        k = causal_conv_seq(k, params["k_conv.conv1.weight"], params["k_conv.conv2.weight"], cfg.n_kv_heads)
    if cfg.use_qk_mean and cfg.n_groups == 1:  # attention.py:233-236
        m = 0.5 * (q_pre + k_pre)
        q = q + m
        k = k + m
    elif cfg.use_qk_mean:  # attention.py:237-246
        q_mean = q_pre.reshape(B, S, cfg.n_heads, hd).mean(dim=2)
        k_mean = k_pre.reshape(B, S, cfg.n_kv_heads, hd).mean(dim=2)
        q = (q.reshape(B, S, cfg.n_heads, hd) + 0.5 * k_mean.unsqueeze(2)).reshape(B, S, L)
        k = (k.reshape(B, S, cfg.n_kv_heads, hd) + 0.5 * q_mean.unsqueeze(2)).reshape(B, S, K)
    q = q.reshape(B, S, cfg.n_heads, hd).transpose(1, 2)  # attention.py:248-250
    k = k.reshape(B, S, cfg.n_kv_heads, hd).transpose(1, 2)
    v = v.reshape(B, S, cfg.n_kv_heads, hd).transpose(1, 2)
    if cfg.use_qk_norm:  # attention.py:260-262
        q = F.normalize(q, p=2, dim=-1)
        k = F.normalize(k, p=2, dim=-1) * params["key_temperature"]
    if cfg.use_rope:  # attention.py:264-266 -> fused_rope / _rope_pytorch
        if cos is None:
            cos, sin = fused_ops.rope_cache(hd, max(S, 1))
        q = fused_ops.rope(q, cos, sin)
        k = fused_ops.rope(k, cos, sin)
    return q.contiguous(), k.contiguous(), v.contiguous()


def attention(q, k, v, *, causal: bool = True, mask=None, scale=None):
    """attention.py:268-327 (CPU branch): padding mask (B,S; 1 = keep) merged
    with the causal mask, K/V expanded to the query heads in
    repeat_interleave order, SDPA."""
    B, Hq, S, hd = q.shape
    G = Hq // k.shape[1]
    attn_mask, is_causal = None, causal
    if mask is not None:
        cm = torch.ones((S, S), dtype=torch.bool).triu(diagonal=1)
        if not causal:
            cm = torch.zeros((S, S), dtype=torch.bool)
        pad = (mask == 0).view(B, 1, 1, S)
        # SDPA boolean masks are "True = attend"; the reference builds
        # "True = masked" (attention.py:276-283) and passes it as attn_mask.
        attn_mask = cm.unsqueeze(0).unsqueeze(0) | pad
        is_causal = False
    k = k.unsqueeze(2).expand(-1, -1, G, -1, -1).reshape(B, Hq, S, hd)
    v = v.unsqueeze(2).expand(-1, -1, G, -1, -1).reshape(B, Hq, S, hd)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=is_causal,
                                          scale=scale)


def attention_bruteforce(q, k, v, *, causal=True, mask=None, scale=None):
    """fp64 triple loop over (b, h, s) with an explicit masked softmax; the
    pin for `attention` on tiny shapes.  A row with no visible key gives 0."""
    B, Hq, S, hd = q.shape
    G = Hq // k.shape[1]
    sc = (1.0 / math.sqrt(hd)) if scale is None else scale
    out = torch.zeros(B, Hq, S, hd, dtype=torch.float64)
    qd, kd, vd = q.double(), k.double(), v.double()
    for b in range(B):
        for h in range(Hq):
            j = h // G
            for s in range(S):
                ts = [t for t in range(S) if (not causal or t <= s) and (mask is None or mask[b, t] != 0)]
                if not ts:
                    continue
                logits = torch.stack([(qd[b, h, s] * kd[b, j, t]).sum() * sc for t in ts])
                p = torch.exp(logits - logits.max())
                p = p / p.sum()
                out[b, h, s] = sum(p[i] * vd[b, j, t] for i, t in enumerate(ts))
    return out


def attention_key_padding(q, k, v, *, causal=True, mask=None, scale=None):
    """The same masked softmax as `attention_bruteforce` (key t visible to
    row s iff (not causal or t <= s) and mask[b, t] != 0; a row with no
    visible key gives 0), vectorised in fp64 for test sizes the triple loop
    cannot reach.  Pinned against `attention_bruteforce`."""
    B, Hq, S, hd = q.shape
    G = Hq // k.shape[1]
    sc = (1.0 / math.sqrt(hd)) if scale is None else scale
    kd = k.double().repeat_interleave(G, 1)
    vd = v.double().repeat_interleave(G, 1)
    logits = (q.double() @ kd.transpose(-1, -2)) * sc
    vis = torch.ones(B, 1, S, S, dtype=torch.bool)
    if causal:
        vis = vis & torch.ones(S, S, dtype=torch.bool).tril()
    if mask is not None:
        vis = vis & (mask != 0).view(B, 1, 1, S)
    logits = logits.masked_fill(~vis, float("-inf"))
    mx = logits.amax(-1, keepdim=True)
    mx = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
    p = torch.exp(logits - mx)
    den = p.sum(-1, keepdim=True)
    p = torch.where(den > 0, p / torch.where(den > 0, den, torch.ones_like(den)), torch.zeros_like(p))
    return p @ vd


def attention_backward(q, k, v, grad_out, *, causal=True, scale=None):
    """fp64 restatement of the split-K backward of CCGQAAttentionFused
    (kernels/fused_attention.py:113-338, :432-635): with P the softmax of
    scale * q k^T (causal: key t visible to query s iff t <= s) recomputed
    from its log-sum-exp, O = P V and D = rowsum(dO * O),
      dV_j = sum_g P_g^T dO_g,  dS = P (dO V^T - D) scale,
      dK_j = sum_g dS_g^T Q_g,  dQ = dS K,
    summing the G = Hq/Hkv query heads g of K/V head j (repeat_interleave
    order) as _bwd_gqa_kv_kernel does.  Returns (dq, dk, dv) in fp64.
    Pinned against autograd through `attention_key_padding`."""
    B, Hq, S, hd = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    sc = (1.0 / math.sqrt(hd)) if scale is None else scale
    qd, dod = q.double(), grad_out.double()
    kd = k.double().repeat_interleave(G, 1)
    vd = v.double().repeat_interleave(G, 1)
    logits = (qd @ kd.transpose(-1, -2)) * sc
    if causal:
        logits = logits.masked_fill(~torch.ones(S, S, dtype=torch.bool).tril(), float("-inf"))
    lse = torch.logsumexp(logits, -1, keepdim=True)
    p = torch.exp(logits - lse)
    o = p @ vd
    d = (dod * o).sum(-1, keepdim=True)
    dv = p.transpose(-1, -2) @ dod
    ds = p * (dod @ vd.transpose(-1, -2) - d) * sc
    dk = ds.transpose(-1, -2) @ qd
    dq = ds @ kd
    dk = dk.view(B, Hkv, G, S, hd).sum(2)
    dv = dv.view(B, Hkv, G, S, hd).sum(2)
    return dq, dk, dv


def forward(params: dict, x: torch.Tensor, cfg: CCGQAConfig, mask=None):
    """CCGQAAttention.forward (attention.py:201-331)."""
    B, S, _ = x.shape
    qkv = F.linear(x, params["qkv_proj.weight"])  # attention.py:205
    q, k, v = prep(params, qkv, cfg)
    # scale=None when QK-norm, else head_dim**-0.5: both are 1/sqrt(head_dim).
    out = attention(q, k, v, causal=True, mask=mask, scale=None)
    out = out.transpose(1, 2).contiguous().view(B, S, cfg.latent_dim)  # attention.py:329
    return F.linear(out, params["o_proj.weight"]) * cfg.output_scale  # attention.py:330


def flops(cfg: CCGQAConfig, B: int, S: int) -> dict:
    """Algorithmic FLOPs of one forward (multiply-add = 2): the figures the
    roofline numbers are computed from."""
    L, K, hd = cfg.latent_dim, cfg.kv_dim, cfg.head_dim
    N = B * S
    ks = cfg.conv_kernel_size
    f = {
        "qkv_proj": 2 * N * cfg.dim * (L + 2 * K),
        "q_conv": 2 * N * ks * (L * hd + L * L) if cfg.use_convs else 0,
        "k_conv": 2 * N * ks * (K * hd + K * K) if cfg.use_convs else 0,
        # causal QK^T + PV including the diagonal: 4 * B * Hq * hd * S(S+1)/2
        "core": 4 * B * cfg.n_heads * hd * S * (S + 1) // 2,
        "o_proj": 2 * N * L * cfg.dim,
    }
    f["total"] = sum(f.values())
    return f
