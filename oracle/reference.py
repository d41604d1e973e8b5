"""fp32 / fp64 restatements of the reference's per-kernel math.

All functions take CPU torch tensors (any float dtype; upcast to fp32 here)
and return fp32 tensors (a tuple for multi-output kernels), unless the name
ends in `_f64`, in which case the arithmetic is float64 throughout.
"""

from __future__ import annotations

import math

import torch

__all__ = [
    "rmsnorm_sum",
    "rmsnorm_weighted",
    "layernorm",
    "softmax_nomax",
    "rope_split",
    "rope_rotate_half",
    "rope_tables",
    "cumsum",
    "cumsum_seq_f32",
    "fused_adam",
    "matmul",
    "rmsnorm_matmul_sum",
    "rmsnorm_matmul_eps",
    "silu_mlp",
    "qkv_cte",
    "softmax_mm",
    "linear_attention",
    "attention_qkv",
    "attention_nomax",
    "attention_causal",
    "ORACLE",
]

NORM_EPS = 1e-6
ADAM_BETA1 = 0.9
ADAM_BETA2 = 0.999
ADAM_EPS = 1e-8


def _f32(*xs):
    return [x.to(torch.float32) for x in xs]


def rmsnorm_sum(x):
    """x / sqrt(sum_j x_j^2) per row; kernels/rmsnorm/refs.py:21-30,
    kernels/rmsnorm/kernel.py:13-20 (sum form, no eps)."""
    (x,) = _f32(x)
    return x / torch.sqrt((x * x).sum(dim=-1, keepdim=True))


def rmsnorm_weighted(x, w, eps=NORM_EPS):
    """x * rsqrt(mean_j x_j^2 + eps) * w; the eps/mean form the reference
    states in kernels/qkv_cte/kernel.py:25-27, with a per-column weight."""
    x, w = _f32(x, w)
    return x * torch.rsqrt((x * x).mean(dim=-1, keepdim=True) + eps) * w


def layernorm(x, eps=NORM_EPS):
    """(x - mean) / sqrt(mean((x - mean)^2) + eps); kernels/layernorm/refs.py:16-37."""
    (x,) = _f32(x)
    d = x - x.mean(dim=-1, keepdim=True)
    return d / torch.sqrt((d * d).mean(dim=-1, keepdim=True) + eps)


def softmax_nomax(x):
    """exp(x) / sum exp(x), no max subtraction; kernels/softmax/kernel.py:13-16,
    kernels/softmax/refs.py:11-13."""
    (x,) = _f32(x)
    e = torch.exp(x)
    return e / e.sum(dim=-1, keepdim=True)


def rope_split(x_even, x_odd, cos, sin):
    """(xe cos - xo sin, xo cos + xe sin); kernels/rope/kernel.py:27-36,
    kernels/rope/refs.py:20-30."""
    xe, xo, c, s = _f32(x_even, x_odd, cos, sin)
    return xe * c - xo * s, xo * c + xe * s


def rope_rotate_half(q, k, cos, sin):
    """Rotate-half RoPE on token-major [b, s, h, d] with cos/sin[s, d]: the
    rotation of kernels/rope/kernel.py:33-36 applied with x_even = x[..., :d/2]
    and x_odd = x[..., d/2:], cos/sin columns taken per output half."""
    q, k, c, s = _f32(q, k, cos, sin)
    half = q.shape[-1] // 2
    c4 = c[None, :, None, :]
    s4 = s[None, :, None, :]

    def rot(x):
        lo, hi = x[..., :half], x[..., half:]
        out_lo = lo * c4[..., :half] - hi * s4[..., :half]
        out_hi = hi * c4[..., half:] + lo * s4[..., half:]
        return torch.cat([out_lo, out_hi], dim=-1)

    return rot(q), rot(k)


def rope_tables(s, d, theta=500000.0):
    """cos/sin[s, d] in fp32 from float64 angles pos * theta^(-2i/d),
    duplicated across the two halves (Llama 3 convention)."""
    inv = theta ** (-(torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = torch.outer(torch.arange(s, dtype=torch.float64), inv)
    emb = torch.cat([ang, ang], dim=-1)
    return torch.cos(emb).to(torch.float32), torch.sin(emb).to(torch.float32)


def cumsum(x):
    """Inclusive prefix sum along the last axis, accumulated in float64 and
    rounded once per element to fp32 (what torch.cumsum does for fp32 on the
    CPU); kernels/cumsum/refs.py:20-22."""
    return torch.cumsum(x.to(torch.float64), dim=-1).to(torch.float32)


def cumsum_seq_f32(x):
    """Sequential fp32 prefix sum (numpy's np.cumsum on fp32,
    kernels/cumsum/refs.py:16-17); kept to show its drift from `cumsum`."""
    (x,) = _f32(x)
    out = torch.empty_like(x)
    acc = torch.zeros(x.shape[:-1], dtype=torch.float32)
    for j in range(x.shape[-1]):
        acc = acc + x[..., j]
        out[..., j] = acc
    return out


def fused_adam(param, grad, exp_avg, exp_avg_sq, step_size, inv_bc2_sqrt, wd):
    """Adam-L2 step with per-row scalars; kernels/fused_adam/refs.py:38-46,
    kernels/fused_adam/kernel.py:20-45. Each operation rounds to fp32."""
    p, g, m, v, ss, ib, w = _f32(param, grad, exp_avg, exp_avg_sq, step_size, inv_bc2_sqrt, wd)
    g2 = g + w * p
    m2 = ADAM_BETA1 * m + (1.0 - ADAM_BETA1) * g2
    v2 = ADAM_BETA2 * v + (1.0 - ADAM_BETA2) * (g2 * g2)
    denom = torch.sqrt(v2) * ib + ADAM_EPS
    return p - m2 / denom * ss, m2, v2


def matmul(x, w):
    """x @ w in fp32; kernels/matmul/refs.py:20-25."""
    x, w = _f32(x, w)
    return x @ w


def rmsnorm_matmul_sum(x, w):
    """(x / sqrt(sum x^2)) @ w; kernels/rmsnorm_matmul/refs.py:16-24."""
    x, w = _f32(x, w)
    return (x / torch.sqrt((x * x).sum(dim=-1, keepdim=True))) @ w


def rmsnorm_matmul_eps(x, w, eps=NORM_EPS):
    """(x * rsqrt(mean x^2 + eps)) @ w; kernels/qkv_cte/refs.py:30-36 without
    the residual sum."""
    x, w = _f32(x, w)
    return (x * torch.rsqrt((x * x).mean(dim=-1, keepdim=True) + eps)) @ w


def silu_mlp(x, w1, w2, w3):
    """(silu(x @ w1) * (x @ w2)) @ w3 with silu(a) = a / (1 + exp(-a));
    kernels/silu_mlp/refs.py:16-22."""
    x, w1, w2, w3 = _f32(x, w1, w2, w3)
    h1 = x @ w1
    return (h1 / (1.0 + torch.exp(-h1)) * (x @ w2)) @ w3


def qkv_cte(x, mlp_prev, attention_prev, w, eps=NORM_EPS):
    """h = (x + mlp_prev) + attention_prev, then (h * rsqrt(mean h^2 + eps)) @ w,
    in fp32; kernels/qkv_cte/kernel.py:18-27, kernels/qkv_cte/refs.py:30-36."""
    x, mlp_prev, attention_prev, w = _f32(x, mlp_prev, attention_prev, w)
    h = (x + mlp_prev) + attention_prev
    return (h * torch.rsqrt((h * h).mean(dim=-1, keepdim=True) + eps)) @ w


def softmax_mm(x, w):
    """(exp(x) / sum_k exp(x)) @ w, bare exp / sum (no max subtraction);
    kernels/softmax_mm/refs.py:16-19, kernels/softmax_mm/kernel.py:7-11."""
    x, w = _f32(x, w)
    e = torch.exp(x)
    return (e / e.sum(dim=-1, keepdim=True)) @ w


def linear_attention(q, key, v):
    """q @ (key^T @ v); kernels/linear_attention/refs.py:20-27."""
    q, key, v = _f32(q, key, v)
    return q @ (key.t() @ v)


def attention_qkv(x, w_q, w_k, w_v):
    """q, k, v = x w_q, x w_k, x w_v; softmax(q k^T) v with a bare exp / sum
    softmax and no scale; kernels/attention/refs.py:16-36, kernel.py:7-18."""
    x, w_q, w_k, w_v = _f32(x, w_q, w_k, w_v)
    q, k, v = x @ w_q, x @ w_k, x @ w_v
    e = torch.exp(q @ k.t())
    return (e / e.sum(dim=-1, keepdim=True)) @ v


def attention_nomax(q, k_t, v):
    """softmax(q @ k_t) @ v with a bare exp/sum softmax;
    kernels/attention_nkilib/refs.py:36-47."""
    q, k_t, v = _f32(q, k_t, v)
    e = torch.exp(q @ k_t)
    return (e / e.sum(dim=-1, keepdim=True)) @ v


def attention_causal(q, k, v, chunk=512):
    """softmax(q k^T / sqrt(d), causal) v in fp32 over [b, h, s, d], with the
    row max subtracted; the two products of kernels/attention_nkilib/kernel.py:14-21
    with scale and mask. Query rows are processed in chunks to bound memory."""
    q, k, v = _f32(q, k, v)
    s, d = q.shape[-2], q.shape[-1]
    scale = 1.0 / math.sqrt(d)
    kt = k.transpose(-1, -2).contiguous()
    out = torch.empty_like(q)
    for i0 in range(0, s, chunk):
        i1 = min(s, i0 + chunk)
        sc = torch.matmul(q[..., i0:i1, :], kt) * scale
        rows = torch.arange(i0, i1)[:, None]
        cols = torch.arange(s)[None, :]
        sc = sc.masked_fill(cols > rows, float("-inf"))
        out[..., i0:i1, :] = torch.matmul(torch.softmax(sc, dim=-1), v)
    return out


# spec name -> oracle function (inputs in the spec's input_specs order)
ORACLE = {
    "rmsnorm": rmsnorm_sum,
    "rmsnorm_weighted": rmsnorm_weighted,
    "layernorm": layernorm,
    "softmax": softmax_nomax,
    "rope": rope_split,
    "rope_llama3": rope_rotate_half,
    "cumsum": cumsum,
    "cumsum_probs": cumsum,
    "fused_adam": fused_adam,
    "matmul": matmul,
    "matmul_std002": matmul,
    "rmsnorm_matmul": rmsnorm_matmul_sum,
    "rmsnorm_matmul_eps": rmsnorm_matmul_eps,
    "silu_mlp": silu_mlp,
    "qkv_cte": qkv_cte,
    "softmax_mm": softmax_mm,
    "linear_attention": linear_attention,
    "attention": attention_qkv,
    "attention_nkilib": attention_nomax,
    "attention_causal": attention_causal,
}
