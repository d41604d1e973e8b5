"""References and inputs for `rmsnorm` (kernels/rmsnorm/refs.py:21-34).

`torch_ref` receives fp32 tensors and returns fp32; the harness casts to the
case dtype. Inputs: x ~ N(0, 1), one float64 draw converted to `dtype`."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16


def baseline_op(x):
    return x / np.sqrt(np.sum(x * x, axis=1, keepdims=True))


def torch_ref(x):
    return x / torch.sqrt(torch.sum(x * x, dim=1, keepdim=True))


def make_inputs(*, m, n, dtype=bfloat16, rng):
    return (astype(rng.standard_normal((m, n)), dtype),)
