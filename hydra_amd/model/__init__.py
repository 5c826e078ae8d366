"""hydra_amd.model -- the block and model compositions of
hydra/model/framework over this package's kernels."""
