"""Oracle for Mixture-of-Depths hard routing
(hydra/routing/mixture_of_depths.py:159-216, hydra/routing/ops.py:257-314,
hydra/model/framework/blocks.py:243-269).

Integer/index work is restated in numpy; the row arithmetic in torch CPU.
Test infrastructure only: see oracle/__init__.py.
"""
from __future__ import annotations

import numpy as np
import torch


def router_k(seq_len: int, capacity_ratio: float) -> int:
    """MoDRouter.forward (mixture_of_depths.py:179-181)."""
    cap = float(min(max(capacity_ratio, 1e-4), 1.0))
    return max(1, min(seq_len, int(seq_len * cap)))


def topk_desc_lowest_index(scores: np.ndarray, k: int) -> np.ndarray:
    """Top-k per row in torch.topk's value order (NaN above +inf, -0.0 ==
    +0.0), ties by ascending index: a stable two-key sort (NaN flag first,
    then the negated value).

    torch.topk (mixture_of_depths.py:187) fixes the value sequence; the tie
    rule (lowest index first) is the one the MoD path is specified with."""
    s = np.asarray(scores, dtype=np.float64)
    nan = np.isnan(s)
    neg = np.where(nan, 0.0, -s)
    neg = np.where(neg == 0.0, 0.0, neg)  # fold -0.0 into +0.0
    # np.lexsort is stable; the last key is the primary one.
    order = np.lexsort((neg, ~nan), axis=-1)
    return order[:, :k].astype(np.int64)


def topk_desc_bruteforce(scores, k: int):
    """Pure-Python selection (repeatedly take the max, lowest index on ties)
    for tiny rows: the pin of topk_desc_lowest_index."""
    out = []
    for row in scores:
        vals = [float(v) for v in row]
        taken = [False] * len(vals)
        sel = []
        for _ in range(k):
            best = None
            for i, v in enumerate(vals):
                if taken[i]:
                    continue
                if best is None:
                    best = i
                    continue
                bv = vals[best]
                if (np.isnan(v) and not np.isnan(bv)) or (not np.isnan(bv) and v > bv):
                    best = i
            taken[best] = True
            sel.append(best)
        out.append(sel)
    return np.array(out, dtype=np.int64)


def sorted_indices(idx_desc: np.ndarray) -> np.ndarray:
    """torch.sort(indices) ascending (blocks.py:261)."""
    return np.sort(idx_desc, axis=-1)


def mask_from_indices(idx: np.ndarray, L: int) -> np.ndarray:
    """mask.scatter_(1, idx, 1.0) (mixture_of_depths.py:190-191)."""
    m = np.zeros((idx.shape[0], L), dtype=np.float32)
    np.put_along_axis(m, idx, 1.0, axis=1)
    return m


def gather(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """gather_by_indices (ops.py:257-272)."""
    return torch.gather(x, 1, idx.unsqueeze(-1).expand(-1, -1, x.shape[-1]))


def residual_scatter(h: torch.Tensor, y: torch.Tensor, idx: torch.Tensor, w=None) -> torch.Tensor:
    """h + zeros_like(h).scatter_(1, idx, y) (blocks.py:266-268 and the
    residual add at :603); with weights: h + scatter(w * y) in fp32, rounded
    once."""
    D = h.shape[-1]
    ix = idx.unsqueeze(-1).expand(-1, -1, D)
    if w is None:
        upd = torch.zeros_like(h).scatter_(1, ix, y.to(h.dtype))
        return h + upd
    hf = h.float()
    upd = torch.zeros_like(hf).scatter_(1, ix, y.float() * w.float().unsqueeze(-1))
    return (hf + upd).to(h.dtype)


def replace_scatter(x: torch.Tensor, y: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """x.clone().scatter_(1, idx, y) (mixture_of_depths.py:291-295)."""
    return x.clone().scatter_(1, idx.unsqueeze(-1).expand(-1, -1, x.shape[-1]), y.to(x.dtype))


def make_tied_logits(B: int, L: int, frac: float, generator: torch.Generator) -> torch.Tensor:
    """Config-4 router logits: fp32 N(0,1) [B, L]; in each row floor(frac*L)
    positions receive the value of another random position of the same row,
    so ties occur (lowest index must win)."""
    s = torch.randn(B, L, generator=generator)
    n = int(frac * L)
    for b in range(B):
        dst = torch.randperm(L, generator=generator)[:n]
        src = torch.randint(0, L, (n,), generator=generator)
        s[b, dst] = s[b, src]
    return s
