"""CPU oracle for the Hyena mixer hot path -- TEST INFRASTRUCTURE ONLY.

A restatement, in plain PyTorch on the CPU, of evo2_flash's reference torch
path for the Hyena mixers (each function cites the reference file:line it
follows).  It is the checker the HIP kernels are compared against, and the
CPU baseline bench.py times beside the GPU.  Only `tests/`,
`__graft_entry__.smoke()` and bench.py's `cpu_baseline` leg may import it;
the product package `evo2_flash_amd` never does and has no CPU fallback.

Pinning: every function here is checked in tests/test_oracle.py against
closed forms, float64 brute force or invariants chosen so that a dropped
term, a flipped tap order or a wrong index fails (impulse responses,
chunk-split and continuation invariance, the sequential recurrence, small
integer known answers).  No function is "parity unpinned" except where the
docstring says so.
"""

from .hyena_ref import *  # noqa: F401,F403
