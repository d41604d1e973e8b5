"""GPU parity driver shared by the test_gpu_* modules: launch a spec's HIP
family through the C ABI for a set of tile tuples and compare each output
with the oracle on the same seeded inputs."""

from __future__ import annotations

from itertools import product

import torch

import oracle
from enzyme_amd import hip
from enzyme_amd.candidate_filter import select_diverse
from tests._specs import as_tuple, spec_inputs, to_device


def legal_tiles(name, variant, dims, codes, n_tiles, options=(1, 2, 4, 8, 16, 32)):
    out = []
    for t in product(options, repeat=n_tiles):
        if hip.check(name, variant, t, dims, codes)[0] == hip.AXON_OK:
            out.append(t)
    return out


def check_parity(name, sizes, *, rtol, atol, variants=None, budget=0, dtype=None,
                 want=None, seed=42, tiles=None):
    """Returns the number of (variant, tiles) keys checked; raises on the first
    mismatch (message names the key). `tiles` names one tile tuple to check
    (it must be legal in every listed variant) instead of the legal set."""
    spec, dims, host = spec_inputs(name, sizes, dtype=dtype, seed=seed)
    dev = to_device(host)
    codes = [hip.dtype_code(t) for t in dev]
    dvals = [dims[d] for d in spec.dim_vars]
    if want is None:
        want = as_tuple(oracle.ORACLE[name](*[t.cpu() for t in dev]))
    explicit = variants is not None
    variants = range(hip.variant_count(name)) if variants is None else variants
    checked = 0
    only = tiles
    for v in variants:
        tiles = legal_tiles(name, v, dvals, codes, len(spec.tile_args))
        if only is not None:
            assert tuple(only) in tiles, f"{name} v{v}: tiles {tuple(only)} are not legal for {sizes}"
            tiles = [tuple(only)]
        # A variant may not serve every shape (hw variant 2 of the plain GEMM
        # needs k % 64 == 0); asked for explicitly, it must.
        if not tiles and not explicit:
            continue
        assert tiles, f"{name} v{v}: no legal tile tuple for {sizes}"
        if budget:
            tiles = select_diverse(tiles, budget=budget, seed=42)
        for t in tiles:
            ln = hip.Launcher(name, v, t, dvals, dev, input_shapes=spec.input_shapes(dims))
            for o in ln.outputs:
                o.fill_(float("nan"))
            ln.launch()
            torch.cuda.synchronize()
            for i, (got, ref) in enumerate(zip(ln.outputs, want)):
                g = got.float().cpu()
                assert torch.isfinite(g).all(), f"{name} v{v} tiles {t} out{i}: non-finite"
                torch.testing.assert_close(
                    g, ref.float(), rtol=rtol, atol=atol,
                    msg=lambda m, v=v, t=t, i=i: f"{name} v{v} tiles {t} out{i}: {m}",
                )
            checked += 1
    assert checked, f"{name}: no hw variant has a legal tile tuple for {sizes}"
    return checked


def silu_mlp_bound(x, w1, w2, w3, ref):
    """Elementwise error bound for silu_mlp's bf16 output at unscaled inputs:
    the bf16 rounding of the output (2^-8 |ref|) plus 2^-14 of the last dot
    product's scale S = sqrt((h * h) @ (w3 * w3)), h = silu(x @ w1) * (x @ w2),
    all in float64 from the given inputs. The kernel's measured excess over
    2^-8 |ref| at the 1024^4 case is below 7e-6 S."""
    x, w1, w2, w3 = (t.detach().cpu().double() for t in (x, w1, w2, w3))
    a = x @ w1
    h = a / (1.0 + torch.exp(-a)) * (x @ w2)
    return 2.0**-8 * ref.detach().cpu().double().abs() + 2.0**-14 * torch.sqrt((h * h) @ (w3 * w3))


def assert_within(got, ref, bound, what):
    """|got - ref| <= bound elementwise (float64 on the host); names the worst
    element on failure."""
    err = (got.detach().cpu().double() - ref.detach().cpu().double()).abs()
    worst = int(torch.argmax(torch.nan_to_num(err - bound, nan=float("inf"))))
    assert bool((err <= bound).all()), (
        f"{what}: |err| {err.flatten()[worst].item():.4g} > bound {bound.flatten()[worst].item():.4g} "
        f"at flat index {worst}")

