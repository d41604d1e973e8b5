"""AxonArray statement of `attention` (the reference's kernels/attention/kernel.py:7-18)."""

from axon import AxonArray


def kernel_attention(x: AxonArray, w_q: AxonArray, w_k: AxonArray, w_v: AxonArray) -> AxonArray:
    q = x @ w_q
    k = x @ w_k
    v = x @ w_v
    e = (q @ k.transpose()).exp()
    return (e / e.sum(axis=1, keep_dims=True)) @ v
