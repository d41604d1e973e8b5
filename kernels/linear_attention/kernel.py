"""AxonArray statement of `linear_attention` (the reference's
kernels/linear_attention/kernel.py:14-20): state = keyᵀ v, out = q state."""

from axon import AxonArray


def kernel_linear_attention(q: AxonArray, key: AxonArray, v: AxonArray) -> AxonArray:
    state = key.transpose() @ v
    return q @ state
