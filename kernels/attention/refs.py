"""References and inputs for `attention` (the reference's
kernels/attention/refs.py: baseline_op 16-25, torch_ref 28-36, make_inputs
39-49): x ~ N(0,1)[m, k]; w_q, w_k ~ N(0,1)[k, n] / (sqrt(k) n^(1/4)) so the
logits q kᵀ stay O(1) (the softmax has no max subtraction); w_v ~
N(0,1)[k, n] / sqrt(k); drawn in that order."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16


def baseline_op(x, w_q, w_k, w_v):
    q, k, v = np.matmul(x, w_q), np.matmul(x, w_k), np.matmul(x, w_v)
    e = np.exp(np.matmul(q, k.T))
    return np.matmul(e / np.sum(e, axis=1, keepdims=True), v)


def torch_ref(x, w_q, w_k, w_v):
    q, k, v = torch.matmul(x, w_q), torch.matmul(x, w_k), torch.matmul(x, w_v)
    e = torch.exp(torch.matmul(q, k.transpose(0, 1)))
    return torch.matmul(e / torch.sum(e, dim=1, keepdim=True), v)


def make_inputs(*, m, n, k, dtype=bfloat16, rng):
    qk_scale = 1.0 / (np.sqrt(k) * n**0.25)
    x = rng.standard_normal((m, k))
    w_q = rng.standard_normal((k, n)) * qk_scale
    w_k = rng.standard_normal((k, n)) * qk_scale
    w_v = rng.standard_normal((k, n)) * (1.0 / np.sqrt(k))
    return astype(x, dtype), astype(w_q, dtype), astype(w_k, dtype), astype(w_v, dtype)
