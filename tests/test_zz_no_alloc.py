"""axon_variant_launch_noalloc (the entry point that allocates nothing; its
workspace is the library's static per-GPU array) against
axon_variant_launch with a caller workspace. Both run the same kernels, so
the outputs must agree bit for bit. Each workload makes two no-alloc calls in
a row, the second on a smaller input, and the single-pass scan runs after a
split-K GEMM has left its partials in the shared array (the scan's slots must
be cleared first). A workload that needs more than the array holds is refused
and enqueues nothing."""

import pytest
import torch

from enzyme_amd import hip
from tests._specs import spec_inputs, to_device

pytestmark = pytest.mark.gpu

# spec, hw variant, tiles, first sizes, second (smaller) sizes; the split-K
# GEMMs run first so the scans find the array holding other data.
CASES = [
    ("matmul_std002", 1, (2, 2, 8), (1024, 512, 16384), (256, 128, 4096)),
    ("rmsnorm_matmul_eps", 0, (2, 2, 8), (1024, 512, 16384), (256, 256, 8192)),
    ("cumsum_probs", 2, (8, 4), (64, 128256), (7, 20000)),
    ("cumsum", 1, (4, 2), (128, 32768), (3, 1001)),
]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


def _launchers(name, variant, tiles, sizes, noalloc):
    spec, dims, host = spec_inputs(name, sizes)
    dev = to_device(host)
    ln = hip.Launcher(name, variant, tiles, [dims[d] for d in spec.dim_vars], dev,
                      input_shapes=spec.input_shapes(dims), noalloc=noalloc)
    for o in ln.outputs:
        o.fill_(float("nan"))
    return ln


@pytest.mark.parametrize("name,variant,tiles,big,small", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_workspace_launch(name, variant, tiles, big, small):
    print(f"noalloc {name} v{variant} tiles {tiles}: {big} then {small}", flush=True)
    assert hip.workspace_bytes(name, variant, tiles, big, _codes(name)) > 0
    na = [_launchers(name, variant, tiles, s, noalloc=True) for s in (big, small)]
    ws = [_launchers(name, variant, tiles, s, noalloc=False) for s in (big, small)]
    assert all(ln.workspace is None for ln in na)
    for ln in na:  # two no-alloc calls in a row, the second smaller
        ln.launch()
    for ln in ws:
        ln.launch()
    torch.cuda.synchronize()
    for a, b, s in zip(na, ws, (big, small)):
        for i, (x, y) in enumerate(zip(a.outputs, b.outputs)):
            assert torch.isfinite(x).all(), f"{name} {s} out{i}: non-finite"
            assert torch.equal(x, y), f"{name} {s} out{i}: differs from the workspace launch"


def _codes(name):
    return [hip.AXON_F32] if name.startswith("cumsum") else [hip.AXON_BF16, hip.AXON_BF16]


def test_noalloc_refuses_oversized_workspace():
    m, n, k = 16384, 512, 8192
    tiles = (4, 4, 16)
    codes = [hip.AXON_BF16] * 4
    need = hip.workspace_bytes("qkv_cte", 2, tiles, (m, n, k), codes)
    assert need > 32 << 20
    dev = [torch.empty(s, dtype=torch.bfloat16, device="cuda") for s in ((m, k), (m, k), (m, k), (k, n))]
    ln = hip.Launcher("qkv_cte", 2, tiles, (m, n, k), dev, noalloc=True)
    ln.outputs[0].fill_(float("nan"))
    with pytest.raises(hip.HipLibraryError) as e:
        ln.launch()
    assert e.value.status == hip.AXON_EWORKSPACE
    assert str(need) in str(e.value)
    torch.cuda.synchronize()
    assert torch.isnan(ln.outputs[0]).all()
