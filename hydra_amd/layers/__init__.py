"""hydra_amd.layers -- the fused-op call sites of hydra/layers/common.py."""
from .common import AdaRMSNorm, RMSNorm, RotaryEmbedding, SwiGLUMLP, SwiGLUMLPFused, residual_norm

__all__ = ["AdaRMSNorm", "RMSNorm", "RotaryEmbedding", "SwiGLUMLP", "SwiGLUMLPFused", "residual_norm"]
