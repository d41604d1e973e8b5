"""AxonArray statement of `cumsum` (kernels/cumsum/kernel.py:12-13)."""

from axon import AxonArray


def kernel_cumsum(x: AxonArray) -> AxonArray:
    return x.cumsum(axis=-1)
