"""ctypes access to oracle/liboracle.so (the C restatement): TEST
INFRASTRUCTURE ONLY. Functions take and return numpy arrays."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB = None
_P = np.ctypeslib.ndpointer


def lib():
    global _LIB
    if _LIB is None:
        path = Path(__file__).resolve().parent / "liboracle.so"
        if not path.is_file():
            from oracle.build import build

            build()
        h = ctypes.CDLL(str(path))
        f32 = _P(np.float32, flags="C_CONTIGUOUS")
        f64 = _P(np.float64, flags="C_CONTIGUOUS")
        i64 = ctypes.c_int64
        h.oracle_cumsum_rows.argtypes = [f32, f32, i64, i64]
        h.oracle_rmsnorm_rows.argtypes = [f32, f32, f32, i64, i64, ctypes.c_int, ctypes.c_double]
        h.oracle_layernorm_rows.argtypes = [f32, f32, i64, i64, ctypes.c_double]
        h.oracle_softmax_rows.argtypes = [f32, f32, i64, i64]
        h.oracle_rope_rotate_half.argtypes = [f32, f32, f32, f32, i64, i64, i64, i64]
        h.oracle_fused_adam.argtypes = [f32] * 10 + [i64, i64]
        h.oracle_matmul_f64.argtypes = [f32, f32, f64, i64, i64, i64]
        h.oracle_attention_head_f64.argtypes = [f32, f32, f32, f64, i64, i64, ctypes.c_double, ctypes.c_int]
        _LIB = h
    return _LIB


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def cumsum(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_cumsum_rows(x, y, x.shape[0], x.shape[1])
    return y


def rmsnorm(x, w=None, eps=1e-6):
    x = _f32(x)
    y = np.empty_like(x)
    ww = _f32(w) if w is not None else np.zeros(x.shape[1], np.float32)
    lib().oracle_rmsnorm_rows(x, ww, y, x.shape[0], x.shape[1], 0 if w is None else 1, eps)
    return y


def layernorm(x, eps=1e-6):
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_layernorm_rows(x, y, x.shape[0], x.shape[1], eps)
    return y


def softmax(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_softmax_rows(x, y, x.shape[0], x.shape[1])
    return y


def rope(x, cos, sin):
    """x [b, s, h, d] token-major."""
    x = _f32(x)
    y = np.empty_like(x)
    b, s, h, d = x.shape
    lib().oracle_rope_rotate_half(x, _f32(cos), _f32(sin), y, b * s, s, h, d)
    return y


def fused_adam(p, g, m, v, step, ibc, wd):
    p, g, m, v = (_f32(a) for a in (p, g, m, v))
    step, ibc, wd = (_f32(a).reshape(-1) for a in (step, ibc, wd))
    po, mo, vo = np.empty_like(p), np.empty_like(p), np.empty_like(p)
    lib().oracle_fused_adam(p, g, m, v, step, ibc, wd, po, mo, vo, p.shape[0], p.shape[1])
    return po, mo, vo


def matmul_f64(x, w):
    x, w = _f32(x), _f32(w)
    y = np.empty((x.shape[0], w.shape[1]), np.float64)
    lib().oracle_matmul_f64(x, w, y, x.shape[0], w.shape[1], x.shape[1])
    return y


def attention_head_f64(q, k, v, scale, causal):
    q, k, v = _f32(q), _f32(k), _f32(v)
    o = np.empty(q.shape, np.float64)
    lib().oracle_attention_head_f64(q, k, v, o, q.shape[0], q.shape[1], scale, 1 if causal else 0)
    return o
