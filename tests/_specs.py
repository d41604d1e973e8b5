"""Helpers shared by the tests: load spec packages by name, draw seeded
inputs, and move them to the GPU."""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[1]
KERNELS = REPO / "kernels"

_CACHE: dict[str, object] = {}


def load_spec(name: str):
    if name not in _CACHE:
        d = KERNELS / name
        mod_name = f"_test_spec_{name}"
        spec = importlib.util.spec_from_file_location(
            mod_name, d / "__init__.py", submodule_search_locations=[str(d)]
        )
        mod = importlib.util.module_from_spec(spec)
        sys.modules[mod_name] = mod
        spec.loader.exec_module(mod)
        _CACHE[name] = mod.SPEC
    return _CACHE[name]


def spec_inputs(name: str, sizes, dtype=None, seed: int = 42):
    spec = load_spec(name)
    dims = dict(zip(spec.dim_vars, sizes, strict=True))
    kw = {"dtype": dtype} if dtype is not None else {}
    return spec, dims, spec.make_inputs(**dims, **kw, rng=np.random.default_rng(seed))


def to_device(inputs, device="cuda"):
    from enzyme_amd.dtypes import to_torch

    return [to_torch(a).to(device) for a in inputs]


def as_tuple(x):
    return x if isinstance(x, tuple) else (x,)
