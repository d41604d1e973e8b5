"""AxonArray statement of `layernorm` (kernels/layernorm/kernel.py:17-25)."""

from axon import AxonArray

EPS = 1e-6


def kernel_layernorm(x: AxonArray) -> AxonArray:
    inv_n = 1.0 / x.shape[1]
    d = x - x.sum(axis=1, keep_dims=True) * inv_n
    var = (d * d).sum(axis=1, keep_dims=True) * inv_n
    return d / (var + EPS).sqrt()
