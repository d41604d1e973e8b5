"""References and inputs for `layernorm` (kernels/layernorm/refs.py:16-37):
mean-centred, divided by sqrt(population variance + 1e-6); x ~ N(0, 1)."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16

EPS = 1e-6


def baseline_op(x):
    d = x - np.mean(x, axis=1, keepdims=True)
    return d / np.sqrt(np.mean(d * d, axis=1, keepdims=True) + EPS)


def torch_ref(x):
    d = x - torch.mean(x, dim=1, keepdim=True)
    return d / torch.sqrt(torch.mean(d * d, dim=1, keepdim=True) + EPS)


def make_inputs(*, m, n, dtype=bfloat16, rng):
    return (astype(rng.standard_normal((m, n)), dtype),)
