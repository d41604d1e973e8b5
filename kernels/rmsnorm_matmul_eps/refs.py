"""References and inputs for `rmsnorm_matmul_eps`: x = 0.02 N(0,1)[m, k],
then w = 0.02 N(0,1)[k, n], converted to `dtype` (bf16)."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16

EPS = 1e-6
STD = 0.02


def baseline_op(x, w):
    ms = np.mean(x * x, axis=1, keepdims=True)
    return np.matmul(x / np.sqrt(ms + EPS), w)


def torch_ref(x, w):
    return torch.matmul(x * torch.rsqrt(torch.mean(x * x, dim=1, keepdim=True) + EPS), w)


def make_inputs(*, m, n, k, dtype=bfloat16, rng):
    x = STD * rng.standard_normal((m, k))
    w = STD * rng.standard_normal((k, n))
    return astype(x, dtype), astype(w, dtype)
