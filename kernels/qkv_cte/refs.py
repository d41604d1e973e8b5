"""References and inputs for `qkv_cte` (the reference's kernels/qkv_cte/refs.py:
baseline_op 23-27, torch_ref 30-36, make_inputs 39-48): x, mlp_prev and
attention_prev ~ N(0,1)[m, k], then w ~ N(0,1)[k, n] / sqrt(k), drawn in that
order and converted to `dtype` (bf16 unless the case says float32)."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16

EPS = 1e-6


def baseline_op(x, mlp_prev, attention_prev, w):
    h = x + mlp_prev + attention_prev
    rms = np.sqrt(np.mean(np.square(h), axis=1, keepdims=True) + EPS)
    return np.matmul(h / rms, w)


def torch_ref(x, mlp_prev, attention_prev, w):
    h = x + mlp_prev + attention_prev
    return torch.matmul(h / torch.sqrt(torch.mean(h * h, dim=1, keepdim=True) + EPS), w)


def make_inputs(*, m, n, k, dtype=bfloat16, rng):
    x = rng.standard_normal((m, k))
    mlp_prev = rng.standard_normal((m, k))
    attention_prev = rng.standard_normal((m, k))
    w = rng.standard_normal((k, n)) / np.sqrt(k)
    return astype(x, dtype), astype(mlp_prev, dtype), astype(attention_prev, dtype), astype(w, dtype)
