"""References and inputs for `rope_llama3`.

Draw order: q ~ N(0,1) [b, s, hq, d], then k ~ N(0,1) [b, s, hkv, d], both
converted to `dtype`. cos/sin are not drawn: with
inv_freq = theta^(-(0, 2, ..., d-2)/d), theta = 500000, and positions
0..s-1, emb = concat(pos (x) inv_freq, pos (x) inv_freq) in float64, then
cos(emb), sin(emb) rounded to float32 [s, d]."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16

ROPE_THETA = 500000.0


def rope_tables(s, d, theta=ROPE_THETA):
    inv_freq = theta ** (-(np.arange(0, d, 2, dtype=np.float64) / d))
    freqs = np.outer(np.arange(s, dtype=np.float64), inv_freq)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def _rotate_half_np(x):
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def baseline_op(q, k, cos, sin):
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    return q * c + _rotate_half_np(q) * s, k * c + _rotate_half_np(k) * s


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def torch_ref(q, k, cos, sin):
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    return (q * c + _rotate_half(q) * s, k * c + _rotate_half(k) * s)


def make_inputs(*, b, s, hq, hkv, d, dtype=bfloat16, rng):
    q = rng.standard_normal((b, s, hq, d))
    k = rng.standard_normal((b, s, hkv, d))
    cos, sin = rope_tables(s, d)
    return astype(q, dtype), astype(k, dtype), cos, sin
