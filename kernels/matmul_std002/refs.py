"""References and inputs for `matmul_std002`: a = 0.02 N(0,1)[m, k], then
b = 0.02 N(0,1)[k, n], converted to `dtype` (bf16)."""

import numpy as np

from axon.dtypes import astype, bfloat16

STD = 0.02


def baseline_op(a, b):
    return np.matmul(a, b)


def torch_ref(a, b):
    return a @ b


def make_inputs(*, m, n, k, dtype=bfloat16, rng):
    a = STD * rng.standard_normal((m, k))
    b = STD * rng.standard_normal((k, n))
    return astype(a, dtype), astype(b, dtype)
