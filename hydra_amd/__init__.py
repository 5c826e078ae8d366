"""hydra_amd -- MI355X (gfx950) implementation of HYDRA's hot path.

Mirrors the reference's Python surface for that path:
  hydra_amd.kernels    fused_rms_norm / fused_rope / fused_swiglu / fused_qk_norm
  hydra_amd.attention  CCGQAAttention, backend registry ("ccgqa"/"ccqa"), factory
  hydra_amd.routing    MoDRouter, MixtureOfDepthsBlock, gather/scatter helpers
  hydra_amd.layers     RMSNorm / SwiGLUMLPFused modules over the fused ops
All compute runs in hand-written HIP kernels (libhydra_amd.so, C ABI in
include/hydra_amd.h); the GEMMs of the projections stay on torch (hipBLASLt).
"""

__version__ = "0.1.0"

from . import _lib  # noqa: F401
