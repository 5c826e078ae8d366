"""Forward-only guard: outputs of the HIP forward kernels carry a grad_fn
whose backward raises, so a training graph through this build fails loudly
instead of silently receiving no gradient."""
from __future__ import annotations

import torch


class _ForwardOnly(torch.autograd.Function):
    @staticmethod
    def forward(ctx, out, *inputs):
        return out.view_as(out)

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(
            "hydra_amd: backward kernels are not part of this build (forward only)")


def track(out: torch.Tensor, *inputs) -> torch.Tensor:
    tensors = [t for t in inputs if isinstance(t, torch.Tensor)]
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        return _ForwardOnly.apply(out, *tensors)
    return out
