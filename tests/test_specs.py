"""Spec packages: KernelSpec validation, three-way agreement of each
package's kernel.py (AxonArray, float64), torch_ref and baseline_op on
seeded inputs, draw order of make_inputs, and the bf16 host conversion."""

import dataclasses

import numpy as np
import pytest
import torch

from axon.kernel_spec import SEED, KernelSpec
from enzyme_amd.axon_array import evaluate
from enzyme_amd.dtypes import astype, to_f32_numpy, to_f32_torch
from tests._specs import KERNELS, load_spec, spec_inputs

SMALL = {
    "rmsnorm": (8, 64), "rmsnorm_weighted": (8, 64), "layernorm": (8, 64), "softmax": (8, 64),
    "rope": (4, 16), "rope_llama3": (1, 8, 4, 2, 16), "cumsum": (4, 50), "cumsum_probs": (4, 50),
    "fused_adam": (4, 16), "matmul": (8, 4, 16), "matmul_std002": (8, 4, 16),
    "rmsnorm_matmul": (8, 4, 16), "rmsnorm_matmul_eps": (8, 4, 16), "silu_mlp": (8, 4, 16, 6),
    "qkv_cte": (8, 4, 16), "softmax_mm": (8, 4, 16), "linear_attention": (8, 12, 4, 6),
    "attention": (8, 4, 16), "attention_nkilib": (16, 8), "attention_causal": (1, 2, 16, 8),
}


def test_every_package_is_listed():
    assert sorted(SMALL) == sorted(p.name for p in KERNELS.iterdir() if (p / "__init__.py").is_file())


@pytest.mark.parametrize("name", sorted(SMALL))
def test_kernel_refs_and_baseline_agree(name):
    spec, dims, ins = spec_inputs(name, SMALL[name])
    t = spec.torch_ref(*[to_f32_torch(a) for a in ins])
    b = spec.baseline_op(*[to_f32_numpy(a) for a in ins])
    a = evaluate(spec.axon_kernel, *ins)
    t = t if isinstance(t, tuple) else (t,)
    b = b if isinstance(b, tuple) else (b,)
    assert len(t) == len(b) == len(a)
    for x, y, z in zip(t, b, a):
        assert torch.allclose(x.double(), torch.as_tensor(np.asarray(y, np.float64)), rtol=1e-5, atol=1e-6)
        assert torch.allclose(x.double(), z, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name", sorted(SMALL))
def test_make_inputs_is_seeded_and_shaped(name):
    spec, dims, a = spec_inputs(name, SMALL[name])
    _, _, b = spec_inputs(name, SMALL[name])
    assert [tuple(x.shape) for x in a] == [tuple(s) for s in spec.input_shapes(dims)]
    for x, y in zip(a, b):
        assert np.array_equal(to_f32_numpy(x), to_f32_numpy(y))


def test_draw_order_rmsnorm_weighted():
    _, _, (x, w) = spec_inputs("rmsnorm_weighted", (3, 5))
    rng = np.random.default_rng(SEED)
    x_raw = rng.standard_normal((3, 5))
    w_raw = 1.0 + 0.1 * rng.standard_normal(5)
    assert np.array_equal(to_f32_numpy(x), to_f32_numpy(astype(x_raw, torch.bfloat16)))
    assert np.array_equal(to_f32_numpy(w), to_f32_numpy(astype(w_raw, torch.bfloat16)))


def test_draw_order_fused_adam_and_constants():
    _, _, ins = spec_inputs("fused_adam", (2, 3), dtype=np.float32)
    rng = np.random.default_rng(SEED)
    draws = [rng.standard_normal((2, 3)) for _ in range(3)] + [np.abs(rng.standard_normal((2, 3)))]
    for got, want in zip(ins[:4], draws):
        assert np.array_equal(got, want.astype(np.float32))
    assert np.all(ins[4] == np.float32(1e-3)) and np.all(ins[5] == 1) and np.all(ins[6] == np.float32(0.01))


def test_rope_llama3_tables():
    _, _, (q, k, c, s) = spec_inputs("rope_llama3", (1, 16, 2, 1, 8))
    assert c.dtype == np.float32 and c.shape == (16, 8)
    assert np.array_equal(c[:, :4], c[:, 4:])
    assert np.allclose(c[3, 1], np.cos(3 * 500000.0 ** (-2 / 8)))


def test_cumsum_probs_rows_are_sorted_distributions():
    _, _, (p,) = spec_inputs("cumsum_probs", (3, 1000))
    assert np.all(np.diff(p, axis=1) <= 0)
    assert np.allclose(p.sum(axis=1, dtype=np.float64), 1.0, atol=1e-5)


def test_bf16_conversion_rounding():
    vals = np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 1 + 2**-8 + 2**-30, 3.4e38, 1e-40])
    got = to_f32_numpy(astype(vals, torch.bfloat16))
    # ties to even; the +2^-30 case rounds to 1.0 because the float32 step
    # lands exactly on the tie first (the float64 -> float32 -> bf16 chain);
    # 3.4e38 rounds past bf16's largest finite value to inf; 1e-40 stays subnormal.
    assert got[0] == 1.0 and got[1] == 1 + 2 * 2**-7 and got[2] == -1.0 and got[3] == 1.0
    assert np.isinf(got[4]) and 0 < got[5] < 1.2e-38


def test_kernelspec_validation():
    spec = load_spec("rmsnorm")
    with pytest.raises(ValueError, match="does not match"):
        dataclasses.replace(spec, dim_vars=("m", "k"))
    with pytest.raises(ValueError, match="duplicate"):
        KernelSpec(name="x", axon_kernel=None, dim_vars=("m", "m"), input_specs=(("x", ("m",)),),
                   make_inputs=None, tile_args=())


def test_draw_order_qkv_cte():
    """x, mlp_prev, attention_prev, then w / sqrt(k), from one generator
    (kernels/qkv_cte/refs.py:39-48 of the reference)."""
    _, _, (x, mp, ap, w) = spec_inputs("qkv_cte", (3, 2, 5), dtype="float32")
    rng = np.random.default_rng(42)
    want = [rng.standard_normal((3, 5)) for _ in range(3)] + [rng.standard_normal((5, 2)) / np.sqrt(5)]
    for got, raw in zip((x, mp, ap, w), want):
        assert np.array_equal(to_f32_numpy(got), raw.astype(np.float32))
