"""Every case of eval/sizes.json (the reference's case list for the specs this
backend serves), every hw variant that serves it, two diverse legal tile
tuples each, against the spec's own torch_ref run in fp32 on the GPU on the
same seeded inputs (the reference's rule: case_gen.py:190-226 coerces inputs
to fp32; bench_runner.py:703-717 compares with np.allclose). Tolerance: the
case's rtol/atol; a case without one (a bench-only case in the reference) is
held to rtol = atol = 1e-2, except silu_mlp sq1k: its unscaled N(0, 1)
inputs give outputs up to ~1e5, where a uniform absolute 1e-2 is below the
rounding of the fp32 intermediate, so it is held elementwise to the bf16
output rounding plus 2^-14 of the last dot product's scale
(tests/_gpu.py silu_mlp_bound). Cases whose
inputs exceed 2^28 elements are covered by the dedicated tests of their
family at full size (test_gpu_qkv.py, test_gpu_composite.py) and skipped
here to keep the input generation short."""

import json

import numpy as np
import pytest
import torch

from enzyme_amd import hip
from enzyme_amd.candidate_filter import select_diverse
from tests._gpu import assert_within, legal_tiles, silu_mlp_bound
from tests._specs import REPO, as_tuple, load_spec, spec_inputs, to_device

pytestmark = pytest.mark.gpu

CASES = json.loads((REPO / "eval" / "sizes.json").read_text())
PARAMS = [(name, cid) for name, per in CASES.items() if not name.startswith("_")
          for cid in per if not cid.startswith("_")]
MAX_ELEMS = 1 << 28


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


def _torch_ref_gpu(spec, dev):
    args = [t.float() for t in dev]
    with torch.no_grad(), torch.device("cuda"):
        return as_tuple(spec.torch_ref(*args))


@pytest.mark.parametrize(("name", "cid"), PARAMS, ids=[f"{n}-{c}" for n, c in PARAMS])
def test_reference_case(name, cid):
    case = CASES[name][cid]
    spec = load_spec(name)
    dims = dict(zip(spec.dim_vars, case["sizes"]))
    elems = sum(int(np.prod(shape)) for shape in spec.input_shapes(dims))
    if elems > MAX_ELEMS:
        pytest.skip(f"{elems} input elements; covered at full size by the family's own tests")
    stated = "rtol" in case
    _, _, host = spec_inputs(name, tuple(case["sizes"]), dtype=case.get("dtype"))
    dev = to_device(host)
    codes = [hip.dtype_code(t) for t in dev]
    dvals = [dims[d] for d in spec.dim_vars]
    want = _torch_ref_gpu(spec, dev)
    bound = None
    if stated:
        rtol, atol = case["rtol"], case["atol"]
    elif name == "silu_mlp":
        bound = silu_mlp_bound(*dev, want[0])
    else:
        rtol, atol = 1e-2, 1e-2
    checked = 0
    for v in range(hip.variant_count(name)):
        tiles = legal_tiles(name, v, dvals, codes, len(spec.tile_args), options=spec.tile_options)
        for t in select_diverse(tiles, budget=2, seed=42) if tiles else []:
            ln = hip.Launcher(name, v, t, dvals, dev, input_shapes=spec.input_shapes(dims))
            for o in ln.outputs:
                o.fill_(float("nan"))
            ln.launch()
            torch.cuda.synchronize()
            for i, (got, ref) in enumerate(zip(ln.outputs, want)):
                if bound is not None:
                    assert_within(got, ref, bound, f"{name}/{cid} v{v} tiles {t} out{i}")
                    continue
                torch.testing.assert_close(got.float(), ref.float(), rtol=rtol, atol=atol,
                                           msg=lambda m, v=v, t=t, i=i: f"{name}/{cid} v{v} tiles {t} out{i}: {m}")
            checked += 1
    assert checked, f"{name}/{cid}: no hw variant serves this case"
