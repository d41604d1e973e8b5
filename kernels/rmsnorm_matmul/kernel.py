"""AxonArray statement of `rmsnorm_matmul` (kernels/rmsnorm_matmul/kernel.py:7-16)."""

from axon import AxonArray


def kernel_rmsnorm_matmul(x: AxonArray, w: AxonArray) -> AxonArray:
    return (x / (x * x).sum(axis=1, keep_dims=True).sqrt()) @ w
