"""References and inputs for `silu_mlp` (kernels/silu_mlp/refs.py:16-30):
silu(a) = a / (1 + exp(-a)); x, w1, w2, w3 ~ N(0,1) drawn in that order."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16


def baseline_op(x, w1, w2, w3):
    h1 = np.matmul(x, w1)
    h2 = np.matmul(x, w2)
    return np.matmul(h1 / (1 + np.exp(-h1)) * h2, w3)


def torch_ref(x, w1, w2, w3):
    h1 = torch.matmul(x, w1)
    h2 = torch.matmul(x, w2)
    return torch.matmul(h1 / (1 + torch.exp(-h1)) * h2, w3)


def make_inputs(*, m, n, k, p, dtype=bfloat16, rng):
    return (
        astype(rng.standard_normal((m, k)), dtype),
        astype(rng.standard_normal((k, n)), dtype),
        astype(rng.standard_normal((k, n)), dtype),
        astype(rng.standard_normal((n, p)), dtype),
    )
