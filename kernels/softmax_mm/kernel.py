"""AxonArray statement of `softmax_mm` (the reference's kernels/softmax_mm/kernel.py:7-11)."""

from axon import AxonArray


def kernel_softmax_matmul(x: AxonArray, w: AxonArray) -> AxonArray:
    e = x.exp()
    return (e / e.sum(axis=1, keep_dims=True)) @ w
