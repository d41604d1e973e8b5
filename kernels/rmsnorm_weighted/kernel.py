"""AxonArray statement of `rmsnorm_weighted`: mean of squares via sum * (1/n),
the same idiom the reference uses for its eps forms (kernels/qkv_cte/kernel.py:25-27)."""

from axon import AxonArray

EPS = 1e-6


def kernel_rmsnorm_weighted(x: AxonArray, weight: AxonArray) -> AxonArray:
    ms = (x * x).sum(axis=1, keep_dims=True) * (1.0 / x.shape[1])
    return x / (ms + EPS).sqrt() * weight
