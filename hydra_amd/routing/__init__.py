"""hydra_amd.routing -- Mixture-of-Depths and Mixture-of-Recursions routing
(hydra/routing/__init__.py: the MoD and MoR names; MoE is not built)."""
from .base import BaseRouter
from .mixture_of_depths import MixtureOfDepthsBlock, MoDMLPWrapper, MoDRouter
from .mixture_of_recursions import MoRConfig, MoRExecutor, MoROutput, MoRRouter
from .ops import (compute_capacity_k, gather_by_indices, mod_topk, router_k,
                  scatter_add_by_indices, scatter_replace, weighted_residual_scatter)

__all__ = [
    "BaseRouter", "MoDRouter", "MixtureOfDepthsBlock", "MoDMLPWrapper",
    "MoRConfig", "MoRRouter", "MoRExecutor", "MoROutput",
    "compute_capacity_k", "router_k", "mod_topk", "gather_by_indices",
    "scatter_add_by_indices", "weighted_residual_scatter", "scatter_replace",
]
