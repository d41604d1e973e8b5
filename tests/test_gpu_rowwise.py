"""GPU parity for the row-resident family (rmsnorm, rmsnorm_weighted,
layernorm, softmax): every legal tile tuple at the reference's case shapes,
the RMSNorm config shape, and ragged shapes, through the C ABI, against the
oracle. Tolerances: bf16 outputs rtol = atol = 1e-2 (the cases' own
tolerance, eval/sizes.json); fp32 softmax rtol = atol = 1e-5."""

from itertools import product

import pytest
import torch

import oracle
from enzyme_amd import hip
from tests._specs import as_tuple, spec_inputs, to_device

pytestmark = pytest.mark.gpu

ROW_CASES = [
    # (spec, sizes, rtol, atol)
    ("rmsnorm", (1024, 1024), 1e-2, 1e-2),
    ("rmsnorm", (1024, 4096), 1e-2, 1e-2),
    ("rmsnorm", (128, 8192), 1e-2, 1e-2),
    ("rmsnorm", (37, 1000), 1e-2, 1e-2),
    ("rmsnorm", (3, 4100), 1e-2, 1e-2),
    ("rmsnorm", (1, 8), 1e-2, 1e-2),
    ("rmsnorm_weighted", (2048, 4096), 1e-2, 1e-2),
    ("rmsnorm_weighted", (19, 777), 1e-2, 1e-2),
    ("layernorm", (128, 8192), 1e-2, 1e-2),
    ("layernorm", (128, 5120), 1e-2, 1e-2),
    ("layernorm", (33, 300), 1e-2, 1e-2),
    ("softmax", (1024, 1024), 1e-5, 1e-6),
    ("softmax", (70, 333), 1e-5, 1e-6),
]


def _legal_tiles(name, dims, codes, options=(1, 2, 4, 8, 16, 32)):
    out = []
    for t in product(options, repeat=2):
        st, _ = hip.check(name, 0, t, dims, codes)
        if st == hip.AXON_OK:
            out.append(t)
    return out


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


@pytest.mark.parametrize(("name", "sizes", "rtol", "atol"), ROW_CASES,
                         ids=[f"{c[0]}-{'x'.join(map(str, c[1]))}" for c in ROW_CASES])
def test_rowwise_parity_all_legal_tiles(name, sizes, rtol, atol):
    spec, dims, host = spec_inputs(name, sizes)
    dev = to_device(host)
    codes = [hip.dtype_code(t) for t in dev]
    dvals = [dims[d] for d in spec.dim_vars]
    want = as_tuple(oracle.ORACLE[name](*[torch.as_tensor(t.float().cpu()) for t in dev]))
    tiles = _legal_tiles(name, dvals, codes)
    assert tiles, "no legal tile tuple"
    for t in tiles:
        ln = hip.Launcher(name, 0, t, dvals, dev, input_shapes=spec.input_shapes(dims))
        for o in ln.outputs:
            o.fill_(float("nan"))
        ln.launch()
        torch.cuda.synchronize()
        for got, ref in zip(ln.outputs, want):
            g = got.float().cpu()
            assert torch.isfinite(g).all(), f"tiles {t}: non-finite output"
            torch.testing.assert_close(g, ref, rtol=rtol, atol=atol, msg=lambda m: f"tiles {t}: {m}")
