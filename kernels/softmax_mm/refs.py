"""References and inputs for `softmax_mm` (the reference's
kernels/softmax_mm/refs.py: baseline_op 16-19, make_inputs 22-26):
x ~ N(0,1)[m, k], then w ~ N(0,1)[k, n], converted to `dtype` (bf16 default)."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16


def baseline_op(a, b):
    e = np.exp(a)
    return np.matmul(e / np.sum(e, axis=1, keepdims=True), b)


def torch_ref(a, b):
    e = torch.exp(a)
    return torch.matmul(e / torch.sum(e, dim=1, keepdim=True), b)


def make_inputs(*, m, n, k, dtype=bfloat16, rng):
    x = rng.standard_normal((m, k))
    w = rng.standard_normal((k, n))
    return astype(x, dtype), astype(w, dtype)
