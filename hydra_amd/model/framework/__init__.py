"""hydra_amd.model.framework -- HydraBlock, HydraMoRBlock, HydraModel
(hydra/model/framework/blocks.py, model.py)."""
from ...routing.mixture_of_depths import MoDMLPWrapper
from .blocks import HydraBlock, HydraMoRBlock
from .model import HydraModel, embedding_lookup

CCGQABlock = HydraBlock
CCGQAMoRBlock = HydraMoRBlock

__all__ = ["HydraBlock", "HydraMoRBlock", "HydraModel", "MoDMLPWrapper", "CCGQABlock",
           "CCGQAMoRBlock", "embedding_lookup"]
