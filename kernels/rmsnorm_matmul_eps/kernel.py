"""AxonArray statement of `rmsnorm_matmul_eps`."""

from axon import AxonArray

EPS = 1e-6


def kernel_rmsnorm_matmul_eps(x: AxonArray, w: AxonArray) -> AxonArray:
    ms = (x * x).sum(axis=1, keep_dims=True) * (1.0 / x.shape[1])
    return (x / (ms + EPS).sqrt()) @ w
