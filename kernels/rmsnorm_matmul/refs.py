"""References and inputs for `rmsnorm_matmul` (kernels/rmsnorm_matmul/refs.py:16-30):
x ~ N(0,1)[m, k], then w ~ N(0,1)[k, n]."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16


def baseline_op(x, w):
    return np.matmul(x / np.sqrt(np.sum(x * x, axis=1, keepdims=True)), w)


def torch_ref(x, w):
    return torch.matmul(x / torch.sqrt(torch.sum(x * x, dim=1, keepdim=True)), w)


def make_inputs(*, m, n, k, dtype=bfloat16, rng):
    return (
        astype(rng.standard_normal((m, k)), dtype),
        astype(rng.standard_normal((k, n)), dtype),
    )
