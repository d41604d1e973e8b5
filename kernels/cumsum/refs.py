"""References and inputs for `cumsum` (kernels/cumsum/refs.py:16-26).

`baseline_op` is numpy's sequential cumsum in the input precision (the
reference's correctness oracle); `torch_ref` is torch.cumsum, which on the
CPU accumulates fp32 rows in double and rounds each prefix once.
Inputs: x ~ N(0, 1), fp32 by default."""

import numpy as np
import torch

from axon.dtypes import astype


def baseline_op(a):
    return np.cumsum(a, axis=-1)


def torch_ref(x):
    return torch.cumsum(x, dim=-1)


def make_inputs(*, m, n, dtype=np.float32, rng):
    return (astype(rng.standard_normal((m, n)), dtype),)
