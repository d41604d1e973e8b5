"""References and inputs for `attention_nkilib` (kernels/attention_nkilib/refs.py:36-65).

Inputs are uniform [0, 1): q [s, d] (times the softmax scale: 1 for d < 512,
0.5 for d >= 512), then k_t [d, s], then v [s, d]."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16


def baseline_op(q, k_t, v):
    e = np.exp(np.matmul(q, k_t))
    return np.matmul(e / np.sum(e, axis=1, keepdims=True), v)


def torch_ref(q, k_t, v):
    e = torch.exp(torch.matmul(q, k_t))
    return torch.matmul(e / torch.sum(e, dim=1, keepdim=True), v)


def softmax_scale(d):
    return 0.5 if d >= 512 else 1.0


def make_inputs(*, s, d, dtype=bfloat16, rng):
    q = rng.random((s, d)) * softmax_scale(d)
    k_t = rng.random((d, s))
    v = rng.random((s, d))
    return astype(q, dtype), astype(k_t, dtype), astype(v, dtype)
