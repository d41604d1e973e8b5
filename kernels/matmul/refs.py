"""References and inputs for `matmul` (kernels/matmul/refs.py:20-38):
x = N(0,1)[m, k] / sqrt(k), w = N(0,1)[k, n], drawn in that order."""

import numpy as np

from axon.dtypes import astype, bfloat16


def baseline_op(x, w):
    return np.matmul(x, w)


def torch_ref(x, w):
    return x @ w


def make_inputs(*, m, n, k, dtype=bfloat16, rng):
    x = rng.standard_normal((m, k)) * (1.0 / np.sqrt(k))
    w = rng.standard_normal((k, n))
    return astype(x, dtype), astype(w, dtype)
