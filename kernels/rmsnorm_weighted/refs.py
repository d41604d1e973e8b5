"""References and inputs for `rmsnorm_weighted`.

Inputs (drawn in this order from the seeded generator):
  x      ~ N(0, 1)        [m, n]
  weight ~ 1 + 0.1 N(0,1) [n]
both converted to `dtype` (bf16 by default)."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16

EPS = 1e-6


def baseline_op(x, weight):
    ms = np.mean(x * x, axis=1, keepdims=True)
    return x / np.sqrt(ms + EPS) * weight


def torch_ref(x, weight):
    return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + EPS) * weight


def make_inputs(*, m, n, dtype=bfloat16, rng):
    x = rng.standard_normal((m, n))
    weight = 1.0 + 0.1 * rng.standard_normal(n)
    return astype(x, dtype), astype(weight, dtype)
