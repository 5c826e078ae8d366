"""CPU oracle of the HYDRA hot path -- TEST INFRASTRUCTURE ONLY.

A restatement, op for op, of the reference's PyTorch CPU path (mcpirate17/HYDRA)
for the fused RMSNorm / RoPE / SwiGLU / QK-norm ops, the CCGQA attention
forward and the Mixture-of-Depths hard routing.  Every function cites the
reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline).  The
product (hydra_amd) never imports it and never falls back to it.

Pinning (what keeps the oracle itself honest) lives in tests/test_oracle_pins.py:
closed forms, brute-force fp64 loops on tiny inputs, library identities, the
reference's own equivalence tests restated, and the golden vectors written by
running the reference (tests/golden/make_golden.py).  No function here is
"parity unpinned".
"""

from . import ccgqa, fused_ops, mod  # noqa: F401
