"""AxonArray statement of `qkv_cte` (the reference's kernels/qkv_cte/kernel.py:18-27)."""

from axon import AxonArray

EPS = 1e-6


def kernel_qkv_cte(x: AxonArray, mlp_prev: AxonArray, attention_prev: AxonArray,
                   w: AxonArray) -> AxonArray:
    h = x + mlp_prev + attention_prev
    ms = (h * h).sum(axis=1, keep_dims=True) * (1.0 / x.shape[1])
    return (h / (ms + EPS).sqrt()) @ w
