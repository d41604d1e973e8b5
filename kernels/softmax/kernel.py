"""AxonArray statement of `softmax` (kernels/softmax/kernel.py:13-16)."""

from axon import AxonArray


def kernel_softmax(x: AxonArray) -> AxonArray:
    e = x.exp()
    return e / e.sum(axis=1, keep_dims=True)
