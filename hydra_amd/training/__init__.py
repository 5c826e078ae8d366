"""hydra_amd.training -- the loss helper of hydra/training/loop.py that the
routing losses use."""
from .loop import compute_token_losses_from_hidden

__all__ = ["compute_token_losses_from_hidden"]
