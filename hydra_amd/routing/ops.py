"""Mixture-of-Depths routing ops on gfx950 (hydra/routing/ops.py:257-314,
mixture_of_depths.py:179-191, model/framework/blocks.py:243-269)."""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _lib
from .._autograd import track


def compute_capacity_k(seq_len: int, capacity_ratio: float) -> int:
    """ops.py:300-314: k = int(L * ratio) clamped to [1, L]."""
    k = int(seq_len * capacity_ratio)
    return max(1, min(seq_len, k))


def router_k(seq_len: int, capacity_ratio: float) -> int:
    """MoDRouter.forward's k (mixture_of_depths.py:179-181): the ratio is
    first clamped to [1e-4, 1]."""
    cap = float(min(max(capacity_ratio, 1e-4), 1.0))
    return max(1, min(seq_len, int(seq_len * cap)))


def mod_topk(scores: torch.Tensor, k: int, *, want_desc: bool = True, want_sorted: bool = True,
             mask_dtype: Optional[torch.dtype] = None
             ) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Per-row top-k of scores [B, L]: (indices in value-descending order with
    ties to the lower index, the same indices ascending, 0/1 mask [B, L] of
    mask_dtype).  The value sequence equals torch.topk's; ties are resolved
    by lowest index."""
    _lib.require_gpu("mod_topk", scores)
    if scores.dim() != 2:
        raise ValueError("mod_topk: scores must be [B, L]")
    B, L = scores.shape
    if not 1 <= k <= L:
        raise ValueError(f"mod_topk: need 1 <= k <= L, got k={k}, L={L}")
    if scores.stride(-1) != 1:
        scores = scores.contiguous()
    dev = scores.device
    desc = torch.empty((B, k), dtype=torch.int64, device=dev) if want_desc else None
    srt = torch.empty((B, k), dtype=torch.int64, device=dev) if want_sorted else None
    mask = torch.empty((B, L), dtype=mask_dtype, device=dev) if mask_dtype is not None else None
    mcode = _lib.dtype_code(mask) if mask is not None else _lib.F32
    with torch.cuda.device(dev):
        _lib.call("hydra_mod_topk", scores.data_ptr(), B, L, scores.stride(0) if B > 0 else L, k,
                  _lib.ptr(desc), _lib.ptr(srt), _lib.ptr(mask), _lib.dtype_code(scores), mcode,
                  _lib.stream(scores))
    return desc, srt, mask


def _bl_strides(x: torch.Tensor):
    if x.stride(-1) != 1:
        return None
    return x.stride(0), x.stride(1)


def gather_by_indices(x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """ops.py:257-272: out[b, j] = x[b, indices[b, j]] -> [B, k, D].
    Indices outside [0, L) produce zero rows."""
    _lib.require_gpu("gather_by_indices", x, indices)
    B, L, D = x.shape
    k = indices.shape[1]
    if indices.shape[0] != B:
        raise ValueError("gather_by_indices: batch mismatch")
    st = _bl_strides(x)
    if st is None:
        x = x.contiguous()
        st = _bl_strides(x)
    idx = indices.to(torch.int64).contiguous()
    out = torch.empty((B, k, D), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("hydra_mod_gather", x.data_ptr(), idx.data_ptr(), out.data_ptr(), B, L, k, D,
                  st[0], st[1], _lib.dtype_code(x), _lib.stream(x))
    return track(out, x)


def _scatter(output, values, indices, weights, mode):
    _lib.require_gpu("scatter", output, values, indices, weights)
    B, L, D = output.shape
    k = indices.shape[1]
    if values.shape != (B, k, D):
        raise ValueError(f"scatter: values shape {tuple(values.shape)} != {(B, k, D)}")
    if values.dtype != output.dtype:
        values = values.to(output.dtype)
    st = _bl_strides(output)
    if st is None:
        raise ValueError("scatter: output must have unit stride on the last dim (it is written in place)")
    vals = values.contiguous()
    idx = indices.to(torch.int64).contiguous()
    w = None if weights is None else weights.to(torch.float32).contiguous()
    with torch.cuda.device(output.device):
        _lib.call("hydra_mod_scatter", output.data_ptr(), vals.data_ptr(), idx.data_ptr(),
                  _lib.ptr(w), B, L, k, D, st[0], st[1], mode, _lib.dtype_code(output),
                  _lib.stream(output))
    return output


def scatter_add_by_indices(output: torch.Tensor, values: torch.Tensor,
                           indices: torch.Tensor) -> torch.Tensor:
    """ops.py:275-293: output[b, indices[b, j]] += values[b, j], in place.
    Indices must be distinct within a row (as top-k indices are)."""
    return _scatter(output, values, indices, None, _lib.SCATTER_ADD)


def weighted_residual_scatter(residual: torch.Tensor, values: torch.Tensor,
                              indices: torch.Tensor,
                              weights: Optional[torch.Tensor] = None) -> torch.Tensor:
    """residual[b, idx[b, j]] += w[b, j] * values[b, j] in place (w = 1 when
    None): the fused form of `h + zeros_like(h).scatter_(idx, y)` of the MoD
    MLP path (blocks.py:266-268 with the residual add at :603)."""
    return _scatter(residual, values, indices, weights, _lib.SCATTER_ADD)


def scatter_replace(output: torch.Tensor, values: torch.Tensor,
                    indices: torch.Tensor) -> torch.Tensor:
    """output[b, idx[b, j]] = values[b, j] in place (the clone + scatter_ of
    MixtureOfDepthsBlock.forward, mixture_of_depths.py:291-295)."""
    return _scatter(output, values, indices, None, _lib.SCATTER_REPLACE)
