"""Mixture-of-Depths routing ops on gfx950 (hydra/routing/ops.py:257-314,
mixture_of_depths.py:179-191, model/framework/blocks.py:243-300).

The row gather and the scatters are autograd Functions whose backward runs
the same HIP kernels (a gather's gradient is a scatter of the incoming
gradient rows, a scatter's is a gather), so the MoD wrappers train through
them as the reference trains through torch.gather / scatter_."""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _lib


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


def _gather(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    B, L, D = x.shape
    k = idx.shape[1]
    st = _bl_strides(x)
    if st is None:
        x = x.contiguous()
        st = _bl_strides(x)
    out = torch.empty((B, k, D), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("hydra_mod_gather", x.data_ptr(), idx.data_ptr(), out.data_ptr(), B, L, k, D,
                  st[0], st[1], _lib.dtype_code(x), _lib.stream(x))
    return out


def _scatter_raw(output: torch.Tensor, values: Optional[torch.Tensor], idx: torch.Tensor,
                 weights: Optional[torch.Tensor], mode: int) -> torch.Tensor:
    B, L, D = output.shape
    k = idx.shape[1]
    st = _bl_strides(output)
    if st is None:
        raise ValueError("scatter: output must have unit stride on the last dim (it is written in place)")
    vals = None
    if values is not None:
        vals = values.to(output.dtype) if values.dtype != output.dtype else values
        vals = vals.contiguous()
    w = None if weights is None else weights.to(torch.float32).contiguous()
    with torch.cuda.device(output.device):
        _lib.call("hydra_mod_scatter", output.data_ptr(), _lib.ptr(vals), idx.data_ptr(),
                  _lib.ptr(w), B, L, k, D, st[0], st[1], mode, _lib.dtype_code(output),
                  _lib.stream(output))
    return output


def _index(indices: torch.Tensor, B: int, name: str) -> torch.Tensor:
    if indices.dim() != 2 or indices.shape[0] != B:
        raise ValueError(f"{name}: indices must be [B, k] with B = {B}")
    return indices.to(torch.int64).contiguous()


class _GatherRows(torch.autograd.Function):
    """xs = x[b, idx[b, j]]; grad_x = scatter-add of grad_xs into zeros
    (the gradient torch.gather gives)."""

    @staticmethod
    def forward(ctx, x, idx, distinct):
        ctx.save_for_backward(idx)
        ctx.shape, ctx.distinct = x.shape, distinct
        return _gather(x, idx)

    @staticmethod
    def backward(ctx, grad):
        (idx,) = ctx.saved_tensors
        gx = torch.zeros(ctx.shape, dtype=grad.dtype, device=grad.device)
        mode = _lib.SCATTER_ADD if ctx.distinct else _lib.SCATTER_ADD_SEQ
        _scatter_raw(gx, grad.contiguous(), idx, None, mode)
        return gx, None, None


class _ScatterRows(torch.autograd.Function):
    """In-place row scatter into `output` (marked dirty):
    ADD: output[b, idx] += w * values -> grad_output = g, grad_values = w * g[idx],
         grad_w = <g[idx], values>;
    REPLACE: output[b, idx] = values -> grad_output = g with rows idx cleared,
         grad_values = g[idx];
    ADD_SEQ: output[b, idx] += values, repeats accumulate -> grad_output = g,
         grad_values = g[idx]."""

    @staticmethod
    def forward(ctx, output, values, idx, weights, mode):
        _scatter_raw(output, values, idx, weights, mode)
        ctx.mark_dirty(output)
        ctx.mode = mode
        ctx.save_for_backward(values, idx, weights)
        return output

    @staticmethod
    def backward(ctx, grad):
        values, idx, weights = ctx.saved_tensors
        grad = grad.contiguous()
        g_sel = None
        if ctx.needs_input_grad[1] or (weights is not None and ctx.needs_input_grad[3]):
            g_sel = _gather(grad, idx)
        g_vals = g_w = None
        if ctx.needs_input_grad[1]:
            # the forward adds fmaf(w, v, out) with the fp32 weight: the
            # product takes the fp32 weight and rounds once
            g_vals = g_sel if weights is None else g_sel.float() * weights.float()[..., None]
            g_vals = g_vals.to(values.dtype)
        if weights is not None and ctx.needs_input_grad[3]:
            g_w = (g_sel.float() * values.float()).sum(-1).to(weights.dtype)
        g_out = None
        if ctx.needs_input_grad[0]:
            if ctx.mode == _lib.SCATTER_REPLACE:
                g_out = _scatter_raw(grad.clone(), None, idx, None, _lib.SCATTER_REPLACE)
            else:
                g_out = grad
        return g_out, g_vals, None, g_w, None


def _scatter(output, values, indices, weights, mode):
    _lib.require_gpu("scatter", output, values, indices, weights)
    B, L, D = output.shape
    idx = _index(indices, B, "scatter")
    k = idx.shape[1]
    if values.shape != (B, k, D):
        raise ValueError(f"scatter: values shape {tuple(values.shape)} != {(B, k, D)}")
    if weights is not None and weights.shape != (B, k):
        raise ValueError(f"scatter: weights shape {tuple(weights.shape)} != {(B, k)}")
    if _bl_strides(output) is None:
        raise ValueError("scatter: output must have unit stride on the last dim (it is written in place)")
    if torch.is_grad_enabled() and (output.requires_grad or values.requires_grad
                                    or (weights is not None and weights.requires_grad)):
        return _ScatterRows.apply(output, values, idx, weights, mode)
    return _scatter_raw(output, values, idx, weights, mode)


def gather_by_indices(x: torch.Tensor, indices: torch.Tensor, *,
                      distinct: bool = False) -> torch.Tensor:
    """ops.py:257-272: out[b, j] = x[b, indices[b, j]] -> [B, k, D].
    Differentiable; `distinct=True` (indices known distinct per row, as top-k
    indices are) lets the backward use the parallel scatter.  Indices outside
    [0, L) give zero rows (torch.gather raises; checking would need a host
    synchronisation)."""
    _lib.require_gpu("gather_by_indices", x, indices)
    if x.dim() != 3:
        raise ValueError("gather_by_indices: x must be [B, L, D]")
    idx = _index(indices, x.shape[0], "gather_by_indices")
    if torch.is_grad_enabled() and x.requires_grad:
        return _GatherRows.apply(x, idx, distinct)
    return _gather(x, idx)


def scatter_add_by_indices(output: torch.Tensor, values: torch.Tensor,
                           indices: torch.Tensor) -> torch.Tensor:
    """ops.py:275-293: output[b, indices[b, j]] += values[b, j], in place,
    with torch.scatter_add_'s semantics: repeated indices accumulate (in
    index order, rounded after each add)."""
    return _scatter(output, values, indices, None, _lib.SCATTER_ADD_SEQ)


def weighted_residual_scatter(residual: torch.Tensor, values: torch.Tensor,
                              indices: torch.Tensor,
                              weights: Optional[torch.Tensor] = None) -> torch.Tensor:
    """residual[b, idx[b, j]] += w[b, j] * values[b, j] in place (w = 1 when
    None; idx distinct per row): the fused form of
    `h + zeros_like(h).scatter_(idx, y)` of the MoD MLP path (blocks.py:266-268
    with the residual add at :603)."""
    return _scatter(residual, values, indices, weights, _lib.SCATTER_ADD)


def scatter_replace(output: torch.Tensor, values: torch.Tensor,
                    indices: torch.Tensor) -> torch.Tensor:
    """output[b, idx[b, j]] = values[b, j] in place (idx distinct per row):
    the clone + scatter_ of MixtureOfDepthsBlock.forward
    (mixture_of_depths.py:291-295) and the zeros + scatter_ of
    MoDMLPWrapper._forward_hard (blocks.py:266-268)."""
    return _scatter(output, values, indices, None, _lib.SCATTER_REPLACE)
