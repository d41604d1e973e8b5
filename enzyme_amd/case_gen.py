"""Per-case harness module for an exported winner.

Same contract as src/axon/case_gen.py:30-131 of the reference: the module
exposes a `CASE` dict (name, entry_point, kernel_rel, refs_rel, dtype,
input_names, shape_args, rtol, atol), a `torch_ref` that coerces every
input to fp32 before the spec's reference and casts each output to the case
dtype (case_gen.py:190-226), `make_inputs` seeded with SEED, and
`output_tensors`. Here it additionally exposes `run_winner(device)`, which
launches the sibling winner module on the GPU with its tile values.
"""

from __future__ import annotations

import json
import os
from pathlib import Path

from enzyme_amd.kernel_spec import SEED, KernelSpec

_TEMPLATE = '''"""Per-case harness for {name!r} (kernel {kernel!r}, dtype {dtype!r}).
Written by enzyme_amd.case_gen; regenerate rather than edit."""

import importlib.util as _ilu
import os as _os

import numpy as np
import torch

from enzyme_amd import dtypes as _dt

_SEED = {seed}
_DTYPE = {dtype!r}
_HERE = _os.path.dirname(_os.path.abspath(__file__))
_SPEC_DIR = _os.path.normpath(_os.path.join(_HERE, {spec_rel!r}))
_INPUT_NAMES = {input_names!r}

CASE = {case}


def _load(path, name, search=None):
    spec = _ilu.spec_from_file_location(name, path, submodule_search_locations=search)
    mod = _ilu.module_from_spec(spec)
    import sys as _sys

    _sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


if _os.path.isdir(_SPEC_DIR):
    _SPEC = _load(_os.path.join(_SPEC_DIR, "__init__.py"), "_axon_case_spec_{kernel}", [_SPEC_DIR]).SPEC
else:
    _SPEC = _load(_SPEC_DIR, "_axon_case_spec_{kernel}").SPEC

_torch_dt = torch.bfloat16 if _DTYPE == "bfloat16" else getattr(torch, _DTYPE)


def torch_ref(*data, **tiles):
    del tiles
    out = _SPEC.torch_ref(*[_dt.to_f32_torch(a) for a in data])
    out = out if isinstance(out, tuple) else (out,)
    return {{f"output_{{i}}": t.to(_torch_dt) for i, t in enumerate(out)}}


def make_inputs(**shape_args):
    dims = {{d: shape_args[d] for d in _SPEC.dim_vars}}
    data = _SPEC.make_inputs(**dims, dtype=_dt.resolve(_DTYPE), rng=np.random.default_rng(_SEED))
    out = dict(zip(_INPUT_NAMES, data))
    out.update({{t: int(shape_args[t]) for t in _SPEC.tile_args if t in shape_args}})
    return out


def output_tensors(kernel_input):
    ref = _SPEC.baseline_op(*[_dt.to_f32_numpy(kernel_input[n]) for n in _INPUT_NAMES])
    ref = ref if isinstance(ref, tuple) else (ref,)
    return {{f"output_{{i}}": np.zeros(np.asarray(a).shape, dtype=np.float32) for i, a in enumerate(ref)}}


def run_winner(device="cuda"):
    """Launch the winner module on `device` with the case's inputs and tiles."""
    kmod = _load(_os.path.join(_HERE, CASE["kernel_rel"]), "_axon_case_winner_{kernel}")
    entry = getattr(kmod, CASE["entry_point"])
    args = make_inputs(**CASE["shape_args"])
    data = [_dt.to_torch(args[n]).to(device) for n in _INPUT_NAMES]
    tiles = {{t: args[t] for t in _SPEC.tile_args}}
    return entry(*data, **tiles)
'''


def generate_case_module(
    spec: KernelSpec,
    kernel_path: Path | str,
    dtype: str,
    dest: Path,
    *,
    name: str,
    entry_point: str,
    shape_args: dict[str, int],
    rtol: float,
    atol: float,
) -> None:
    """Write the harness module to `dest` (needs spec.torch_ref and
    spec.baseline_op, as in the reference)."""
    if spec.torch_ref is None or spec.baseline_op is None:
        raise ValueError(
            f"{spec.name}: head-to-head case needs both spec.torch_ref and spec.baseline_op"
        )
    kabs = Path(kernel_path).resolve()
    dest = Path(dest).resolve()
    rel = os.path.relpath(kabs, dest.parent)
    names = [n for n, _ in spec.input_specs]
    for label, group in (("input", names), ("dim", list(spec.dim_vars)), ("tile", list(spec.tile_args))):
        bad = [n for n in group if not n.isidentifier()]
        if bad:
            raise ValueError(f"{spec.name}: {label} names are not valid identifiers: {bad}")
    case = {
        "name": name,
        "entry_point": entry_point,
        "kernel_rel": f"{name}.py",
        "refs_rel": os.path.join(rel, "refs.py") if kabs.is_dir() else rel,
        "dtype": dtype,
        "input_names": names,
        "shape_args": shape_args,
        "rtol": rtol,
        "atol": atol,
    }
    dest.parent.mkdir(parents=True, exist_ok=True)
    dest.write_text(
        _TEMPLATE.format(
            name=name,
            kernel=spec.name,
            dtype=dtype,
            seed=SEED,
            spec_rel=rel,
            input_names=names,
            case=json.dumps(case, indent=4),
        )
    )
