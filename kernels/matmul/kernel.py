"""AxonArray statement of `matmul` (kernels/matmul/kernel.py:7-8)."""

from axon import AxonArray


def kernel_matmul(x: AxonArray, w: AxonArray) -> AxonArray:
    return x @ w
