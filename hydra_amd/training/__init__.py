"""hydra_amd.training -- the loss helper of hydra/training/loop.py that the
routing losses use, and loading of the reference's checkpoints."""
from .checkpointing import load_module_from_checkpoint, module_state, read_checkpoint
from .loop import compute_token_losses_from_hidden

__all__ = ["compute_token_losses_from_hidden", "load_module_from_checkpoint", "module_state",
           "read_checkpoint"]
