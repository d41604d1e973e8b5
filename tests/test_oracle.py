"""Pins of the oracle, each independent of the formula it checks:
library routines (F.rms_norm, F.layer_norm, torch.softmax,
torch.optim.Adam, F.scaled_dot_product_attention, complex multiplication),
the float64 C restatement in oracle/csrc, closed forms and invariants.
`test_planted_mistakes_are_caught` plants plausible mistakes in copies of
the oracle and checks that the same pins reject each of them."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import clib
from tests._specs import spec_inputs

torch.manual_seed(0)
RNG = np.random.default_rng(1)


def randn(*shape, scale=1.0):
    return torch.from_numpy(RNG.standard_normal(shape).astype(np.float32) * scale)


# ---- row norms ----------------------------------------------------------
def pin_rmsnorm_sum(fn):
    x = randn(7, 300)
    y = fn(x)
    assert torch.allclose((y.double() ** 2).sum(-1), torch.ones(7, dtype=torch.float64), atol=1e-5)
    assert np.allclose(y.numpy(), clib.rmsnorm(x.numpy()), rtol=1e-5, atol=1e-7)


def pin_rmsnorm_weighted(fn):
    x, w = randn(7, 300), 1 + 0.1 * randn(300)
    ref = F.rms_norm(x, (300,), w, eps=1e-6)
    assert torch.allclose(fn(x, w), ref, rtol=1e-5, atol=1e-6)
    assert np.allclose(fn(x, w).numpy(), clib.rmsnorm(x.numpy(), w.numpy()), rtol=1e-5, atol=1e-7)


def pin_layernorm(fn):
    x = randn(5, 513, scale=3.0) + 2.0
    y = fn(x)
    assert torch.allclose(y, F.layer_norm(x, (513,), eps=1e-6), rtol=1e-5, atol=1e-5)
    assert torch.allclose(y.mean(-1), torch.zeros(5), atol=1e-5)
    assert np.allclose(y.numpy(), clib.layernorm(x.numpy()), rtol=1e-4, atol=1e-5)


def pin_softmax(fn):
    x = randn(6, 257)
    y = fn(x)
    assert torch.allclose(y, torch.softmax(x, -1), rtol=1e-6, atol=1e-8)
    assert np.allclose(y.numpy(), clib.softmax(x.numpy()), rtol=1e-5, atol=1e-9)


# ---- rope -----------------------------------------------------------------
def pin_rope_split(fn):
    xe, xo = randn(8, 33), randn(8, 33)
    ang = torch.from_numpy(RNG.uniform(-math.pi, math.pi, (8, 33)).astype(np.float32))
    c, s = torch.cos(ang), torch.sin(ang)
    oe, oo = fn(xe, xo, c, s)
    z = torch.complex(xe.double(), xo.double()) * torch.complex(c.double(), s.double())
    assert torch.allclose(oe.double(), z.real, atol=1e-5) and torch.allclose(oo.double(), z.imag, atol=1e-5)


def pin_rope_rotate_half(fn):
    b, s, hq, hk, d = 2, 9, 3, 1, 64
    q, k = randn(b, s, hq, d), randn(b, s, hk, d)
    c, sn = oracle.rope_tables(s, d, theta=10000.0)
    oq, ok = fn(q, k, c, sn)
    # (x[i], x[i + d/2]) rotates by the angle pos * theta^(-2i/d).
    half = d // 2
    pos = torch.arange(s, dtype=torch.float64)[:, None]
    ang = pos * 10000.0 ** (-(torch.arange(half, dtype=torch.float64) * 2 / d))[None, :]
    for x, o in ((q, oq), (k, ok)):
        z = torch.complex(x[..., :half].double(), x[..., half:].double())
        z = z * torch.polar(torch.ones_like(ang), ang)[None, :, None, :]
        assert torch.allclose(o[..., :half].double(), z.real, atol=1e-5)
        assert torch.allclose(o[..., half:].double(), z.imag, atol=1e-5)
        assert np.allclose(o.numpy(), clib.rope(x.numpy(), c.numpy(), sn.numpy()), atol=1e-6)
    assert torch.equal(oq[:, 0], q[:, 0])  # position 0: identity


def test_rope_tables_closed_form():
    c, s = oracle.rope_tables(5, 8, theta=500000.0)
    for p in range(5):
        for i in range(4):
            a = p * 500000.0 ** (-2 * i / 8)
            assert c[p, i] == c[p, i + 4] == np.float32(math.cos(a))
            assert s[p, i] == s[p, i + 4] == np.float32(math.sin(a))


# ---- cumsum ---------------------------------------------------------------
def pin_cumsum(fn):
    x = randn(3, 1000)
    y = fn(x)
    assert np.array_equal(y.numpy(), clib.cumsum(x.numpy()))
    for j in (0, 17, 999):
        assert y[1, j].item() == np.float32(math.fsum(x[1, : j + 1].double().tolist()))
    assert torch.equal(y, torch.cumsum(x, -1))  # torch's CPU cumsum accumulates in double


def test_sequential_fp32_baseline_drifts_past_1e5_on_nucleus_input():
    _, _, (probs,) = spec_inputs("cumsum_probs", (2, 128256))
    p = torch.as_tensor(probs)
    ref = oracle.cumsum(p)
    assert ((oracle.cumsum_seq_f32(p) - ref).abs() / ref).max() > 1e-5
    assert abs(ref[:, -1].double() - 1.0).max() < 1e-5  # a probability row sums to 1


# ---- adam -----------------------------------------------------------------
def pin_adam(fn):
    p0, g, m0 = randn(4, 64), randn(4, 64), randn(4, 64)
    v0 = randn(4, 64).abs()
    lr, wd, step = 1e-3, 0.01, 5
    bc1, bc2 = 1 - 0.9 ** (step + 1), 1 - 0.999 ** (step + 1)
    col = lambda v: torch.full((4, 1), v, dtype=torch.float32)  # noqa: E731
    po, mo, vo = fn(p0, g, m0, v0, col(lr / bc1), col(1 / math.sqrt(bc2)), col(wd))
    par = torch.nn.Parameter(p0.clone())
    opt = torch.optim.Adam([par], lr=lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd,
                           foreach=False, fused=False)
    par.grad = g.clone()
    opt.state[par] = {"step": torch.tensor(float(step)), "exp_avg": m0.clone(), "exp_avg_sq": v0.clone()}
    opt.step()
    st = opt.state[par]
    assert torch.allclose(mo, st["exp_avg"], rtol=1e-6, atol=1e-7)
    assert torch.allclose(vo, st["exp_avg_sq"], rtol=1e-6, atol=1e-7)
    assert torch.allclose(po, par.detach(), rtol=1e-5, atol=1e-7)
    # Same op order as the C restatement (built without contraction): bit-equal.
    cp, cm, cv = clib.fused_adam(p0, g, m0, v0, col(lr / bc1), col(1 / math.sqrt(bc2)), col(wd))
    assert np.array_equal(po.numpy(), cp) and np.array_equal(mo.numpy(), cm) and np.array_equal(vo.numpy(), cv)


def test_adam_zero_grad_zero_wd_decays_moments():
    m, v = randn(2, 8), randn(2, 8).abs()
    z = torch.zeros(2, 8)
    col = lambda x: torch.full((2, 1), x)  # noqa: E731
    _, m2, v2 = oracle.fused_adam(randn(2, 8), z, m, v, col(1e-3), col(1.0), col(0.0))
    assert torch.equal(m2, np.float32(0.9) * m) and torch.equal(v2, np.float32(0.999) * v)


# ---- matmul family ------------------------------------------------------------
def pin_matmul(fn):
    x, w = randn(13, 70), randn(70, 9)
    assert np.allclose(fn(x, w).numpy(), clib.matmul_f64(x.numpy(), w.numpy()), rtol=1e-5, atol=1e-5)


def pin_rmsnorm_matmul_sum(fn):
    x, w = randn(13, 70), randn(70, 9)
    ref = clib.matmul_f64(clib.rmsnorm(x.numpy()), w.numpy())
    assert np.allclose(fn(x, w).numpy(), ref, rtol=1e-5, atol=1e-5)


def pin_rmsnorm_matmul_eps(fn):
    x, w = randn(13, 70, scale=0.02), randn(70, 9, scale=0.02)
    ref = F.rms_norm(x, (70,), eps=1e-6) @ w
    assert torch.allclose(fn(x, w), ref, rtol=1e-5, atol=1e-6)


def pin_silu_mlp(fn):
    x, w1, w2, w3 = randn(6, 16), randn(16, 24, scale=0.25), randn(16, 24, scale=0.25), randn(24, 5)
    ref = (F.silu(x.double() @ w1.double()) * (x.double() @ w2.double())) @ w3.double()
    assert torch.allclose(fn(x, w1, w2, w3).double(), ref, rtol=1e-5, atol=1e-5)


def pin_qkv_cte(fn):
    # Small magnitudes so eps (1e-6) moves the result by about 10%, and three
    # different residual streams, so dropping any one of them fails.
    x, mp, ap = randn(11, 72, scale=1e-3), randn(11, 72, scale=2e-3), randn(11, 72, scale=3e-3)
    w = randn(72, 9)
    h = x.double() + mp.double() + ap.double()
    ref = F.rms_norm(h, (72,), eps=1e-6) @ w.double()
    assert torch.allclose(fn(x, mp, ap, w).double(), ref, rtol=1e-5, atol=1e-6)
    # The C restatement: weighted RMSNorm (unit weight, eps 1e-6) of the
    # summed stream, then the float64 product.
    cref = clib.matmul_f64(clib.rmsnorm(h.float().numpy(), np.ones(72, np.float32)), w.numpy())
    assert np.allclose(fn(x, mp, ap, w).numpy(), cref, rtol=1e-5, atol=1e-6)
    # The row scale is invariant to scaling h when eps is negligible.
    big = [t * 1e3 for t in (x, mp, ap)]
    assert torch.allclose(fn(*big, w), fn(*[t * 2e3 for t in (x, mp, ap)], w), rtol=1e-4, atol=1e-5)


def pin_softmax_mm(fn):
    x, w = randn(9, 40), randn(40, 7)
    ref = torch.softmax(x.double(), dim=-1) @ w.double()
    assert torch.allclose(fn(x, w).double(), ref, rtol=1e-5, atol=1e-6)
    # Each output row is a convex combination of the rows of w.
    out = fn(x, torch.eye(40))
    assert torch.allclose(out.sum(-1), torch.ones(9), atol=1e-5) and bool((out > 0).all())


def pin_linear_attention(fn):
    sq, sk, dk, dv = 12, 20, 8, 6
    q, key, v = torch.rand(sq, dk), torch.rand(sk, dk), torch.rand(sk, dv)
    # Evaluated the other way round, (q key^T) v, by the float64 C product.
    scores = clib.matmul_f64(q.numpy(), key.t().contiguous().numpy())
    ref = scores @ v.double().numpy()
    assert np.allclose(fn(q, key, v).numpy(), ref, rtol=1e-5, atol=1e-5)
    # Brute force on a tiny case: out[i][c] = sum_j (q_i . key_j) v[j][c].
    bf = [[sum(float(q[i] @ key[j]) * float(v[j][c]) for j in range(sk)) for c in range(dv)] for i in range(2)]
    assert np.allclose(fn(q, key, v)[:2].numpy(), np.array(bf), rtol=1e-5, atol=1e-5)


def pin_attention_qkv(fn):
    m, n, k = 24, 16, 32
    x = randn(m, k)
    w_q, w_k, w_v = randn(k, n, scale=0.1), randn(k, n, scale=0.1), randn(k, n, scale=0.2)
    xd = x.double()
    q, kk, v = xd @ w_q.double(), xd @ w_k.double(), xd @ w_v.double()
    ref = F.scaled_dot_product_attention(q[None], kk[None], v[None], scale=1.0)[0]
    assert torch.allclose(fn(x, w_q, w_k, w_v).double(), ref, rtol=1e-5, atol=1e-6)
    c = clib.attention_head_f64(q.float().numpy(), kk.float().numpy(), v.float().numpy(), 1.0, False)
    assert np.allclose(fn(x, w_q, w_k, w_v).numpy(), c, rtol=1e-4, atol=1e-5)


# ---- attention ------------------------------------------------------------
def pin_attention_nomax(fn):
    s, d = 40, 16
    q, kt, v = torch.rand(s, d), torch.rand(d, s), torch.rand(s, d)
    ref = F.scaled_dot_product_attention(q[None], kt.t()[None].contiguous(), v[None], scale=1.0)[0]
    assert torch.allclose(fn(q, kt, v), ref, rtol=1e-5, atol=1e-5)
    c = clib.attention_head_f64(q.numpy(), kt.t().contiguous().numpy(), v.numpy(), 1.0, False)
    assert np.allclose(fn(q, kt, v).numpy(), c, rtol=1e-5, atol=1e-6)


def pin_attention_causal(fn):
    b, h, s, d = 2, 3, 37, 16
    q, k, v = randn(b, h, s, d), randn(b, h, s, d), randn(b, h, s, d)
    out = fn(q, k, v)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-5)
    assert torch.allclose(out[..., 0, :], v[..., 0, :])  # the first query sees only key 0
    c = clib.attention_head_f64(q[1, 2].numpy(), k[1, 2].numpy(), v[1, 2].numpy(), 1 / math.sqrt(d), True)
    assert np.allclose(out[1, 2].numpy(), c, rtol=1e-5, atol=1e-6)


PINS = {
    "rmsnorm_sum": pin_rmsnorm_sum,
    "rmsnorm_weighted": pin_rmsnorm_weighted,
    "layernorm": pin_layernorm,
    "softmax_nomax": pin_softmax,
    "rope_split": pin_rope_split,
    "rope_rotate_half": pin_rope_rotate_half,
    "cumsum": pin_cumsum,
    "fused_adam": pin_adam,
    "matmul": pin_matmul,
    "rmsnorm_matmul_sum": pin_rmsnorm_matmul_sum,
    "rmsnorm_matmul_eps": pin_rmsnorm_matmul_eps,
    "silu_mlp": pin_silu_mlp,
    "qkv_cte": pin_qkv_cte,
    "softmax_mm": pin_softmax_mm,
    "linear_attention": pin_linear_attention,
    "attention_qkv": pin_attention_qkv,
    "attention_nomax": pin_attention_nomax,
    "attention_causal": pin_attention_causal,
}


def test_every_oracle_function_has_a_pin():
    used = {fn.__name__ for fn in oracle.ORACLE.values()}
    assert used <= set(PINS)


@pytest.mark.parametrize("name", sorted(PINS))
def test_oracle_pinned(name):
    PINS[name](getattr(oracle, name))


def _mutants():
    """(pin, mutated function) pairs: each mutation is a plausible slip."""
    def sum_to_mean(x):
        return x / torch.sqrt((x * x).mean(-1, keepdim=True))

    def no_eps_no_weight(x, w):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True))

    def ln_sample_var(x):
        d = x - x.mean(-1, keepdim=True)
        return d / torch.sqrt((d * d).sum(-1, keepdim=True) / (x.shape[-1] - 1) + 1e-6)

    def rope_sign(xe, xo, c, s):
        return xe * c + xo * s, xo * c - xe * s

    def rope_same_half(q, k, c, s):
        return oracle.rope_rotate_half(q, k, c, torch.cat([s[:, :32], -s[:, :32]], -1))

    def exclusive_cumsum(x):
        return torch.cumsum(x.double(), -1).float() - x

    def adam_no_wd(p, g, m, v, ss, ib, wd):
        return oracle.fused_adam(p, g, m, v, ss, ib, torch.zeros_like(wd))

    def matmul_transposed(x, w):
        return (w.t() @ x.t()).t() * 1.0001

    def qkv_two_residuals(x, mp, ap, w):
        return oracle.qkv_cte(x, mp, torch.zeros_like(ap), w)

    def qkv_no_eps(x, mp, ap, w):
        return oracle.qkv_cte(x, mp, ap, w, eps=0.0)

    def softmax_mm_columns(x, w):
        e = torch.exp(x)
        return (e / e.sum(dim=0, keepdim=True)) @ w

    def linear_attention_scaled(q, key, v):
        return oracle.linear_attention(q, key, v) / key.shape[0]

    def attention_qkv_scaled(x, w_q, w_k, w_v):
        return oracle.attention_qkv(x, w_q / math.sqrt(w_q.shape[1]), w_k, w_v)

    def attention_qkv_swapped(x, w_q, w_k, w_v):
        return oracle.attention_qkv(x, w_k, w_q, w_v)

    def attn_no_mask(q, k, v):
        return F.scaled_dot_product_attention(q, k, v)

    def attn_no_scale(q, k, v):
        return oracle.attention_causal(q * math.sqrt(q.shape[-1]), k, v)

    return [
        ("rmsnorm_sum", sum_to_mean),
        ("rmsnorm_weighted", no_eps_no_weight),
        ("layernorm", ln_sample_var),
        ("rope_split", rope_sign),
        ("rope_rotate_half", rope_same_half),
        ("cumsum", exclusive_cumsum),
        ("fused_adam", adam_no_wd),
        ("matmul", matmul_transposed),
        ("qkv_cte", qkv_two_residuals),
        ("qkv_cte", qkv_no_eps),
        ("softmax_mm", softmax_mm_columns),
        ("linear_attention", linear_attention_scaled),
        ("attention_qkv", attention_qkv_scaled),
        ("attention_qkv", attention_qkv_swapped),
        ("attention_causal", attn_no_mask),
        ("attention_causal", attn_no_scale),
    ]


@pytest.mark.parametrize(("pin", "mutant"), _mutants(), ids=lambda v: v if isinstance(v, str) else v.__name__)
def test_planted_mistakes_are_caught(pin, mutant):
    with pytest.raises(AssertionError):
        PINS[pin](mutant)
