"""hydra_amd.layers -- the fused-op call sites of hydra/layers/common.py."""
from .common import RMSNorm, SwiGLUMLPFused

__all__ = ["RMSNorm", "SwiGLUMLPFused"]
