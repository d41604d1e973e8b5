"""References and inputs for `linear_attention` (the reference's
kernels/linear_attention/refs.py: baseline_op 20-22, torch_ref 25-27,
make_inputs 30-36): q ~ U[0,1)[sq, dk], key ~ U[0,1)[sk, dk],
v ~ U[0,1)[sk, dv], drawn in that order."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16


def baseline_op(q, key, v):
    return np.matmul(q, np.matmul(key.T, v))


def torch_ref(q, key, v):
    return torch.matmul(q, torch.matmul(key.transpose(-1, -2), v))


def make_inputs(*, sq, sk, dk, dv, dtype=bfloat16, rng):
    q = rng.random((sq, dk))
    key = rng.random((sk, dk))
    v = rng.random((sk, dv))
    return astype(q, dtype), astype(key, dtype), astype(v, dtype)
