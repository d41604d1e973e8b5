"""References and inputs for `cumsum_probs`.

Inputs: logits = 3 * N(0, 1) [m, n] (float64); probs = softmax(logits) per
row in float64, sorted descending, converted to `dtype` (fp32).
Both references accumulate in float64 and round each prefix once to the
output precision, so they agree bit for bit with each other."""

import numpy as np
import torch

from axon.dtypes import astype


def baseline_op(probs):
    return np.cumsum(np.asarray(probs, dtype=np.float64), axis=-1).astype(np.float32)


def torch_ref(probs):
    return torch.cumsum(probs, dim=-1)


def make_inputs(*, m, n, dtype=np.float32, rng):
    logits = 3.0 * rng.standard_normal((m, n))
    z = np.exp(logits - logits.max(axis=-1, keepdims=True))
    probs = z / z.sum(axis=-1, keepdims=True)
    probs = -np.sort(-probs, axis=-1)
    return (astype(probs, dtype),)
