"""AxonArray statement of `rmsnorm` (kernels/rmsnorm/kernel.py:13-20): the
row is divided by the square root of its sum of squares."""

from axon import AxonArray


def kernel_rmsnorm(x: AxonArray) -> AxonArray:
    return x / (x * x).sum(axis=1, keep_dims=True).sqrt()
