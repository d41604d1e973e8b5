"""GPU parity for the bf16 MFMA GEMM family through the C ABI.

Every case compares the bf16 output with the fp32 oracle at rtol = atol =
1e-2 (the bf16 bar), over a diverse selection of legal tile tuples that
includes split-K (partials + fixup kernel) and single-pass schedules, in
both hw variants (one or several K steps of loads in flight), at the
reference's case shapes, the BASELINE shapes (1024 x 512 x 16384) and ragged
shapes (m not a multiple of the tile).

fp32 matmul (hi/lo bf16 planes over K' = 3k, fp32 output) is held to the
reference's fp32 tolerance rtol = atol = 1e-3 at its ck_16k_l2 shape
(1024 x 1024 x 16384) and at ragged shapes.

silu_mlp with the spec's unscaled N(0, 1) inputs has outputs up to ~1e5, so
a uniform absolute 1e-2 is below the rounding of its fp32 intermediate
there. That case is held elementwise to the bf16 output rounding plus a
term on the dot product's own scale: |got - ref| <= 2^-8 |ref| + 2^-14 S,
S = sqrt((h * h) @ (w3 * w3)) with h = silu(x @ w1) * (x @ w2); the kernel's
measured excess over 2^-8 |ref| is below 7e-6 S. A scaled case
(w ~ N(0, 1/fan_in)) is held to the plain 1e-2 / 1e-2."""

import numpy as np
import pytest
import torch

import oracle
from enzyme_amd import hip
from enzyme_amd.dtypes import astype
from tests._gpu import check_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


@pytest.mark.parametrize(
    ("name", "sizes"),
    [
        ("matmul", (1024, 1024, 1024)),
        ("matmul", (100, 72, 200)),
        ("matmul", (1024, 512, 16384)),
        ("matmul_std002", (1024, 512, 16384)),
        ("rmsnorm_matmul", (1024, 1024, 1024)),
        ("rmsnorm_matmul", (77, 136, 520)),
        ("rmsnorm_matmul_eps", (1024, 512, 16384)),
    ],
)
def test_gemm_parity(name, sizes):
    assert check_parity(name, sizes, rtol=1e-2, atol=1e-2, budget=10)


@pytest.mark.parametrize("variant", [0, 1, 3])
def test_gemm_repeated_launches_bit_identical(variant):
    """Split-K launches reuse one workspace: ten launches give the same bits
    every time (the fixup sums the partials in a fixed order)."""
    from tests._specs import spec_inputs, to_device

    spec, dims, host = spec_inputs("matmul_std002", (256, 128, 4096))
    dev = to_device(host)
    ln = hip.Launcher("matmul_std002", variant, (2, 2, 8), [256, 128, 4096], dev)
    ln.launch()
    torch.cuda.synchronize()
    first = ln.outputs[0].clone()
    for _ in range(10):
        ln.launch()
    torch.cuda.synchronize()
    assert torch.equal(first, ln.outputs[0])


def test_silu_mlp_unscaled_elementwise():
    """The spec's sq1k case (N(0, 1) inputs) in every hw variant over a
    diverse tile selection, elementwise against the oracle."""
    from enzyme_amd.candidate_filter import select_diverse
    from tests._gpu import assert_within, legal_tiles, silu_mlp_bound
    from tests._specs import spec_inputs, to_device

    sizes = (1024, 1024, 1024, 1024)
    spec, dims, host = spec_inputs("silu_mlp", sizes)
    dev = to_device(host)
    ref = oracle.silu_mlp(*[t.cpu() for t in dev])
    bound = silu_mlp_bound(*dev, ref)
    codes = [hip.dtype_code(t) for t in dev]
    checked = 0
    for v in range(hip.variant_count("silu_mlp")):
        for t in select_diverse(legal_tiles("silu_mlp", v, list(sizes), codes, 4), budget=6, seed=42):
            ln = hip.Launcher("silu_mlp", v, t, list(sizes), dev)
            ln.outputs[0].fill_(float("nan"))
            ln.launch()
            torch.cuda.synchronize()
            assert_within(ln.outputs[0], ref, bound, f"silu_mlp v{v} tiles {t}")
            checked += 1
    assert checked


def test_silu_mlp_scaled_elementwise():
    from enzyme_amd.dtypes import to_torch

    m, n, k, p = 256, 512, 384, 128
    rng = np.random.default_rng(7)
    x = astype(rng.standard_normal((m, k)), torch.bfloat16)
    w1 = astype(rng.standard_normal((k, n)) / np.sqrt(k), torch.bfloat16)
    w2 = astype(rng.standard_normal((k, n)) / np.sqrt(k), torch.bfloat16)
    w3 = astype(rng.standard_normal((n, p)) / np.sqrt(n), torch.bfloat16)
    ref = oracle.silu_mlp(x, w1, w2, w3)
    dev = [to_torch(t).cuda() for t in (x, w1, w2, w3)]
    from itertools import product

    for tiles in product((1, 2, 4), (1, 2, 4), (1, 2, 8), (1, 2, 4)):
        if hip.check("silu_mlp", 0, tiles, [m, n, k, p], [0, 0, 0, 0])[0] != hip.AXON_OK:
            continue
        ln = hip.Launcher("silu_mlp", 0, tiles, [m, n, k, p], dev)
        ln.launch()
        torch.cuda.synchronize()
        torch.testing.assert_close(ln.outputs[0].float().cpu(), ref, rtol=1e-2, atol=1e-2,
                                   msg=lambda s, t=tiles: f"tiles {t}: {s}")


@pytest.mark.parametrize("sizes", [(1024, 1024, 16384), (100, 72, 200), (33, 520, 1032), (1, 8, 8)])
def test_matmul_fp32(sizes):
    """fp32 x and w through hw variants 0 and 1 (variant 2 has no fp32
    instantiation and is refused)."""
    print(f"matmul fp32 {sizes}", flush=True)
    assert check_parity("matmul", sizes, rtol=1e-3, atol=1e-3, dtype="float32", variants=[0, 1],
                        budget=4 if sizes[2] > 10000 else 8)
    codes = [hip.AXON_F32, hip.AXON_F32]
    assert hip.check("matmul", 2, (1, 1, 1), sizes, codes)[0] == hip.AXON_EDTYPE


@pytest.mark.parametrize(
    ("name", "sizes", "empty_dim"),
    [
        ("matmul", (64, 128, 0), "k"),
        ("rmsnorm_matmul", (64, 128, 0), "k"),
        ("rmsnorm_matmul_eps", (64, 128, 0), "k"),
        ("softmax_mm", (64, 128, 0), "k"),
        ("qkv_cte", (64, 128, 0), "k"),
        ("silu_mlp", (64, 64, 0, 128), "k"),
        ("silu_mlp", (64, 0, 64, 128), "n"),
        ("linear_attention", (64, 0, 128, 64), "sk"),
    ],
)
def test_empty_contraction_gives_zeros(name, sizes, empty_dim):
    """A zero-length contraction with non-empty outputs: the reference's math
    gives zeros (the normalised or softmaxed row is empty). torch gives
    zero-element tensors a null data pointer, which the C ABI refuses with
    AXON_EARG; with valid pointers (larger live buffers, the dims saying the
    contraction is empty) every hw variant writes exact zeros. With no K step
    no kernel reads the operands."""
    from tests._gpu import legal_tiles
    from tests._specs import load_spec

    print(f"empty contraction {name} {sizes}", flush=True)
    spec = load_spec(name)
    dims = dict(zip(spec.dim_vars, sizes))
    shapes = spec.input_shapes(dims)
    live = [torch.randn([max(d, 8) for d in shape], device="cuda").to(torch.bfloat16) for shape in shapes]
    views = [t[tuple(slice(0, d) for d in shape)] for t, shape in zip(live, shapes)]
    want = oracle.ORACLE[name](*[t.cpu() for t in views])
    want = want if isinstance(want, tuple) else (want,)
    assert all(torch.count_nonzero(w) == 0 for w in want)
    codes = [hip.dtype_code(t) for t in live]
    checked = 0
    for v in range(hip.variant_count(name)):
        for tiles in legal_tiles(name, v, list(sizes), codes, len(spec.tile_args))[:2]:
            if any(t.data_ptr() == 0 for t in views):
                with pytest.raises(hip.HipLibraryError) as e:
                    hip.Launcher(name, v, tiles, list(sizes), views).launch()
                assert e.value.status == hip.AXON_EARG and "null" in str(e.value), str(e.value)
            ln = hip.Launcher(name, v, tiles, list(sizes), live)
            for o in ln.outputs:
                o.fill_(float("nan"))
            ln.launch()
            torch.cuda.synchronize()
            for o in ln.outputs:
                assert torch.count_nonzero(o) == 0 and not torch.isnan(o).any(), (name, v, tiles)
            checked += 1
    assert checked
