"""AxonArray statement of `silu_mlp` (kernels/silu_mlp/kernel.py:7-14)."""

from axon import AxonArray


def kernel_silu_mlp_full(x: AxonArray, w1: AxonArray, w2: AxonArray, w3: AxonArray) -> AxonArray:
    return ((x @ w1).silu() * (x @ w2)) @ w3
