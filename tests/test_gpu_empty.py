"""Empty inputs on the GPU through the product launcher: with the leading
dim 0, every family and hw variant allocates empty outputs of the right
shape and launches nothing (the C ABI returns before any kernel or
workspace use)."""

from itertools import product

import pytest
import torch

from enzyme_amd import hip
from enzyme_amd.dtypes import to_torch
from tests._specs import KERNELS, load_spec, spec_inputs

pytestmark = pytest.mark.gpu

# Small legal dims per spec; the first dim is set to 0.
DIMS = {"attention_causal": [1, 2, 64, 128], "attention_nkilib": [64, 128],
        "rope_llama3": [1, 64, 4, 2, 128], "rope": [64, 128]}
NAMES = sorted(p.name for p in KERNELS.iterdir() if (p / "__init__.py").exists())


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


@pytest.mark.parametrize("name", NAMES)
def test_empty_leading_dimension(name):
    print(f"empty {name}", flush=True)
    spec = load_spec(name)
    small = DIMS.get(name, [8] * len(spec.dim_vars))
    _, _, host = spec_inputs(name, tuple(small))
    dtypes = [to_torch(a).dtype for a in host]
    dims = [0] + list(DIMS.get(name, [64] * len(spec.dim_vars)))[1:]
    shapes = spec.input_shapes(dict(zip(spec.dim_vars, dims)))
    inputs = [torch.empty(shape, dtype=dt, device="cuda") for shape, dt in zip(shapes, dtypes)]
    codes = [hip.dtype_code(t) for t in inputs]
    want = hip.outputs(name, dims, codes)
    for v in range(hip.variant_count(name)):
        tiles = next(t for t in product(spec.tile_options, repeat=len(spec.tile_args))
                     if hip.check(name, v, t, dims, codes)[0] == hip.AXON_OK)
        ln = hip.Launcher(name, v, tiles, dims, inputs, input_shapes=shapes)
        ln.launch()
        torch.cuda.synchronize()
        assert [tuple(o.shape) for o in ln.outputs] == [tuple(d.shape) for d in want], (name, v)
        assert all(o.numel() == 0 for o in ln.outputs), (name, v)
