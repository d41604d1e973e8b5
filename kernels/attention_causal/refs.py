"""References and inputs for `attention_causal`.

Draw order: q, k, v ~ N(0, 1) [b, h, s, d], converted to `dtype` (bf16).
Scores q k^T are scaled by 1/sqrt(d); key j > query i is masked out; the
softmax subtracts the row max; all in fp32."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16


def baseline_op(q, k, v):
    d = q.shape[-1]
    s = q.shape[-2]
    scores = np.matmul(q, np.swapaxes(k, -1, -2)) * np.float32(1.0 / np.sqrt(d))
    mask = np.triu(np.ones((s, s), dtype=bool), k=1)
    scores = np.where(mask, np.float32(-np.inf), scores)
    scores = scores - scores.max(axis=-1, keepdims=True)
    e = np.exp(scores)
    return np.matmul(e / e.sum(axis=-1, keepdims=True), v)


def torch_ref(q, k, v):
    d = q.shape[-1]
    s = q.shape[-2]
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * (1.0 / d**0.5)
    mask = torch.ones(s, s, dtype=torch.bool).triu(1)
    scores = scores.masked_fill(mask, float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), v)


def make_inputs(*, b, h, s, d, dtype=bfloat16, rng):
    shape = (b, h, s, d)
    q = rng.standard_normal(shape)
    k = rng.standard_normal(shape)
    v = rng.standard_normal(shape)
    return astype(q, dtype), astype(k, dtype), astype(v, dtype)
