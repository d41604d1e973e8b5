"""The oracle against golden vectors written by tests/golden/make_golden.py
(plain Python float64 loops, independent of the oracle's code)."""

from pathlib import Path

import numpy as np
import torch

import oracle

G = np.load(Path(__file__).resolve().parent / "golden" / "vectors.npz")


def t(name):
    return torch.from_numpy(G[name].astype(np.float32))


def close(got, name, rtol=1e-5, atol=1e-6):
    assert np.allclose(got.double().numpy(), G[name], rtol=rtol, atol=atol), name


def test_norms_softmax_cumsum():
    close(oracle.rmsnorm_sum(t("rms_x")), "rms_sum_y")
    close(oracle.rmsnorm_weighted(t("rms_x"), t("rms_w")), "rms_w_y")
    close(oracle.layernorm(t("rms_x")), "ln_y", atol=1e-5)
    close(oracle.softmax_nomax(t("rms_x")), "softmax_y")
    close(oracle.cumsum(t("rms_x")), "cumsum_y", atol=1e-5)


def test_matmul_and_attention():
    close(oracle.matmul(t("mm_a"), t("mm_b")), "mm_y", atol=1e-5)
    q, k, v = (t(n)[None, None] for n in ("at_q", "at_k", "at_v"))
    close(oracle.attention_causal(q, k, v)[0, 0], "at_causal_y")


def test_rope():
    x = t("rope_x")[None, :, None, :]
    c, s = oracle.rope_tables(3, 8)
    oq, _ = oracle.rope_rotate_half(x, x[:, :, :0], c, s)
    close(oq[0, :, 0], "rope_y", atol=1e-6)
