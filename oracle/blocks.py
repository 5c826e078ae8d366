"""Oracle for the HYDRA block compositions: the config-1 block (embedding +
HydraBlock) and the HydraModel forward (MoR blocks with MoD, tied LM head).
Test infrastructure only: see oracle/__init__.py.

Functional form over the reference's state_dict (keys as
hydra/model/framework/{blocks,model}.py name them), restating the CPU path
op for op:
  _safe_embedding_lookup            model.py:51-73
  RMSNorm.forward (F.rms_norm)      hydra/layers/common.py:90-105
  AdaRMSNorm._rmsnorm               common.py:153-157
  SwiGLUMLPFused.forward            common.py:224-230
  HydraBlock.forward                blocks.py:68-70
  MoDMLPWrapper._forward_hard       blocks.py:243-269 (MoDRouter.forward,
                                    mixture_of_depths.py:159-216)
  MoRRouter.forward                 mixture_of_recursions.py:238-288
  MoRExecutor.forward               mixture_of_recursions.py:370-478
  HydraMoRBlock._forward_mor        blocks.py:614-633
  HydraModel.forward                model.py:408-502
The one choice the reference leaves open: torch.topk's order among tied
router scores; here ties go to the lower index (the rule the build's kernel
implements), through oracle.mod.topk_desc_lowest_index.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import ccgqa, mod


def embedding(table: torch.Tensor, ids: torch.Tensor, scale: float) -> torch.Tensor:
    """model.py:51-73: ids clamped into [0, V), rows times scale."""
    return F.embedding(ids.clamp(0, table.shape[0] - 1), table) * scale


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm module (common.py:104-105): F.rms_norm."""
    return F.rms_norm(x, [x.shape[-1]], weight=w, eps=eps)


def ada_rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """AdaRMSNorm._rmsnorm (common.py:153-157), in x's dtype."""
    rms = x.pow(2).mean(dim=-1, keepdim=True)
    return x * torch.rsqrt(rms + eps) * w


def swiglu_mlp(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor) -> torch.Tensor:
    """SwiGLUMLPFused.forward (common.py:224-230; the CPU branch)."""
    gate, up = F.linear(x, w_gate_up).chunk(2, dim=-1)
    return F.linear(F.silu(gate) * up, w_down)


def _sub(params: dict, prefix: str) -> dict:
    return {k[len(prefix):]: v for k, v in params.items() if k.startswith(prefix)}


def hydra_block(params: dict, x: torch.Tensor, cfg: ccgqa.CCGQAConfig, eps: float = 1e-6) -> torch.Tensor:
    """HydraBlock.forward (blocks.py:68-70): h = x + attn(norm1(x));
    h + mlp(norm2(h)).  params: the block's state_dict (attention.*,
    norm1.weight, norm2.weight, mlp.gate_up.weight, mlp.down.weight)."""
    a = ccgqa.forward(_sub(params, "attention."), rms_norm(x, params["norm1.weight"], eps), cfg)
    h = x + a
    return h + swiglu_mlp(rms_norm(h, params["norm2.weight"], eps), params["mlp.gate_up.weight"],
                          params["mlp.down.weight"])


def c1_forward(params: dict, ids: torch.Tensor, cfg: ccgqa.CCGQAConfig) -> torch.Tensor:
    """Config 1: embedding * sqrt(dim) then HydraBlock (params: the block's
    state_dict plus tok_emb.weight)."""
    h0 = embedding(params["tok_emb.weight"], ids, math.sqrt(cfg.dim))
    return hydra_block(params, h0, cfg)


def mod_mlp_hard(params: dict, x: torch.Tensor, capacity: float, force_idx=None) -> torch.Tensor:
    """MoDMLPWrapper._forward_hard (blocks.py:243-269): router scores
    (Linear(dim, 1)), top-k of k = int(L * cap) (ties to the lower index),
    indices sorted, gathered rows through the MLP, scattered into zeros.
    force_idx: optional [B, k] selection to use instead (a test that checks
    the selection separately feeds the device's own)."""
    B, L, D = x.shape
    scores = F.linear(x, params["mod_router.router.weight"], params["mod_router.router.bias"]).squeeze(-1)
    k = mod.router_k(L, capacity)
    if force_idx is None:
        idx = torch.from_numpy(mod.topk_desc_lowest_index(scores.float().numpy(), k))
    else:
        idx = force_idx
    idx = torch.sort(idx, dim=1).values
    ie = idx.unsqueeze(-1).expand(-1, -1, D)
    y = swiglu_mlp(torch.gather(x, 1, ie), params["mlp.gate_up.weight"], params["mlp.down.weight"])
    out = torch.zeros_like(x)
    out.scatter_(1, ie, y.to(out.dtype))
    return out


def mor_route(logits: torch.Tensor, n_rec: int, min_d: int = 0):
    """MoRRouter.forward after the GEMV (mixture_of_recursions.py:259-288)."""
    logits = torch.tanh(logits / 2.0) * 3.0
    probs = torch.sigmoid(logits)
    if min_d > 0:
        dc = min_d + probs * (n_rec - 1 - min_d)
    else:
        dc = probs * (n_rec - 1)
    depths = torch.clamp(torch.round(dc).long(), min_d, n_rec - 1)
    return depths, probs, logits


def mor_executor(x, depths, probs, mlp_fn, norm_fn, rec_bias, rec_embed, n_rec: int):
    """MoRExecutor.forward (mixture_of_recursions.py:414-478), forward
    values (the straight-through factor is 1)."""
    output = torch.zeros_like(x)
    current = x
    for i in range(n_rec):
        active = (depths >= i).unsqueeze(-1).to(x.dtype)
        exit_ = (depths == i).unsqueeze(-1).to(x.dtype)
        h = current + rec_bias[i].squeeze() + rec_embed[i]
        current = current + mlp_fn(norm_fn(h), i) * active
        output = output + current * exit_
    return output


@dataclass
class ModelConfig:
    """HydraModel constructor arguments the forward depends on."""
    vocab_size: int
    dim: int
    n_mor_blocks: int
    recursions_per_block: int
    n_heads: int
    n_kv_heads: int
    compression_factor: int
    max_seq_len: int
    mod_capacity: float
    mor_min_depth: int = 0
    mod_enabled: bool = True  # set_global_step past the MoD warmup

    def attn_cfg(self) -> ccgqa.CCGQAConfig:
        return ccgqa.CCGQAConfig(dim=self.dim, n_heads=self.n_heads, n_kv_heads=self.n_kv_heads,
                                 compression_factor=self.compression_factor,
                                 max_seq_len=self.max_seq_len)


def hydra_mor_block(params: dict, x: torch.Tensor, cfg: ModelConfig, use_mod: bool,
                    trace: dict | None = None, force: dict | None = None) -> torch.Tensor:
    """HydraMoRBlock._forward_mor (blocks.py:614-633) with AdaRMSNorm
    pre-norms (the default, HYDRA_USE_ADA_RMSNORM=1).  trace (optional)
    receives the routing decisions: "depths" and per recursion "mod_idx{i}";
    force (optional) supplies them instead of computing them."""
    R = cfg.recursions_per_block
    a = ccgqa.forward(_sub(params, "attention."), ada_rms_norm(x, params["norm1.weight"]), cfg.attn_cfg())
    h = x + 0.5 * a
    logits = F.linear(h, params["mor_router.router.weight"], params["mor_router.router.bias"]).squeeze(-1)
    depths, probs, _ = mor_route(logits, R, cfg.mor_min_depth)
    if force is not None and "depths" in force:
        depths = force["depths"]
    if trace is not None:
        trace["depths"] = depths
        trace["router_logits"] = logits

    def mlp_fn(y, i):
        if use_mod and cfg.mod_enabled:
            fi = None if force is None else force.get(f"mod_idx{i}")
            if trace is not None:
                sc = F.linear(y, params["mod_mlp_wrapper.mod_router.router.weight"],
                              params["mod_mlp_wrapper.mod_router.router.bias"]).squeeze(-1)
                trace[f"mod_scores{i}"] = sc
            return mod_mlp_hard(_sub(params, "mod_mlp_wrapper."), y, cfg.mod_capacity, force_idx=fi)
        return swiglu_mlp(y, params["mlp.gate_up.weight"], params["mlp.down.weight"])

    out = mor_executor(h, depths, probs, mlp_fn, lambda t: ada_rms_norm(t, params["norm2.weight"]),
                       params["mor_executor.recursion_bias"], params["mor_executor.recursion_embed.weight"], R)
    return rms_norm(out, params["final_norm.weight"])


def hydra_model(params: dict, ids: torch.Tensor, cfg: ModelConfig, traces: list | None = None,
                forces: list | None = None, return_hidden: bool = False) -> torch.Tensor:
    """HydraModel.forward (model.py:424-502, no MoE): embedding * sqrt(dim),
    the MoR blocks (MoD on blocks 1..n-2, model.py:283), final RMSNorm, LM
    head with the output weight (tied to the embedding in the reference's
    default)."""
    h = embedding(params["tok_emb.weight"], ids, math.sqrt(cfg.dim))
    for i in range(cfg.n_mor_blocks):
        use_mod = 0 < i < cfg.n_mor_blocks - 1
        tr = {} if traces is not None else None
        h = hydra_mor_block(_sub(params, f"layers.{i}."), h, cfg, use_mod, trace=tr,
                            force=None if forces is None else forces[i])
        if traces is not None:
            traces.append(tr)
    h = rms_norm(h, params["norm.weight"])
    if return_hidden:
        return h
    return F.linear(h, params.get("output.weight", params["tok_emb.weight"]))


def flops_c1(cfg: ccgqa.CCGQAConfig, B: int, S: int, hidden: int) -> float:
    """Algorithmic FLOPs of one config-1 block forward: the CCGQA module
    (oracle.ccgqa.flops) plus the SwiGLU GEMMs (gate_up 2*N*D*2H, down
    2*N*H*D)."""
    N = B * S
    return ccgqa.flops(cfg, B, S)["total"] + 2 * N * cfg.dim * 2 * hidden + 2 * N * hidden * cfg.dim


__all__ = ["embedding", "rms_norm", "ada_rms_norm", "swiglu_mlp", "hydra_block", "c1_forward",
           "mod_mlp_hard", "mor_route", "mor_executor", "ModelConfig", "hydra_mor_block",
           "hydra_model", "flops_c1", "np"]
