"""CPU oracle for the HIP kernel set: TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only to check or time against it.
The product path (enzyme_amd, libaxon_hip.so) never calls it: a missing
native library is an error there, never a reason to fall back to this code.

Each function restates, in fp32 torch (the reference's `torch_ref`
convention: inputs upcast to fp32, src/axon/case_gen.py:190-201) or in
float64 numpy, one reference function, and cites the file:line it follows.
How each is pinned independently of its own formula (library routines,
closed forms, invariants, fp64 brute force, golden vectors) is in
tests/test_oracle.py; every function has at least one such pin.
"""

from oracle.reference import *  # noqa: F401,F403
