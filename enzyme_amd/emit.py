"""Write the per-variant modules of a spec from libaxon_hip.so's registry.

This replaces the reference's synthesis + NKI emission (src/axon/cli.py:697-755
writing `out/<stem>/<fn>__v<i>_t<j>.py` via
src/axon/codegen/assemble.py:824-860). Each hw variant of the spec's HIP
family becomes one module `<fn>__v<i>_t0.py` holding

* the literal tile manifest `__axon_tile_constraints__` for the concrete
  sizes (same format as src/axon/candidate_filter.py:48-53);
* a literal `__axon_hip_kernel__` record naming the family, variant, dims
  and target; the compile worker reads it without importing the module;
* one entry function named after the spec whose parameters are the spec's
  input names then its tile args (src/axon/codegen/assemble.py:405-488),
  which launches the instantiation and returns the outputs.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any

from enzyme_amd import dtypes as _dt
from enzyme_amd.candidate_filter import MANIFEST_NAME, manifest_literal
from enzyme_amd.kernel_spec import KernelSpec
from enzyme_amd.paths import RunPaths


def safe_name(node_id: str) -> str:
    """A Python identifier for a spec name (the reference's `nki_safe_var`,
    src/axon/codegen/ops.py:57-62)."""
    out = node_id.replace("-", "_").replace(".", "_").replace("/", "_").lstrip("_")
    if not out or out[0].isdigit():
        out = "v" + out
    return out


# Alias under the reference's name.
nki_safe_var = safe_name

_DTYPE_CODE = {"bfloat16": 0, "float16": 1, "float32": 2}


def input0_dtype_code(spec: KernelSpec, dtype: Any | None) -> int:
    """Element type of the first input: `--dtype` when given, else the
    default of `make_inputs`' `dtype=` parameter (float32 when it has none)."""
    import inspect

    if dtype is not None:
        return _DTYPE_CODE[_dt.dtype_name(dtype)]
    param = inspect.signature(spec.make_inputs).parameters.get("dtype")
    if param is None or param.default is inspect.Parameter.empty:
        return _DTYPE_CODE["float32"]
    return _DTYPE_CODE[_dt.dtype_name(param.default)]


_TEMPLATE = '''"""HIP variant module: spec {name!r}, hw_variant {i}, tile_variant {j}.

{summary}

Written by enzyme_amd.emit for sizes {dims}. The entry `{fn}` runs
libaxon_hip.so's instantiation for the TILES_IN_BLOCK_* values it is called
with; it takes GPU tensors and returns the output tensor(s)."""

from enzyme_amd import hip as _hip

{manifest_name} = {manifest}

{meta_name} = {meta!r}


def {fn}({params}):
    return _hip.run_variant({meta_name}, ({inputs}), ({tiles}))
'''


def variant_module_text(spec: KernelSpec, dim_sizes: dict[str, int], hw_variant: int,
                        tile_variant: int, dtype_code: int, target: str = "gfx950") -> str:
    from enzyme_amd import hip

    desc = hip.describe(spec.name, hw_variant)
    if tuple(desc["tile_args"]) != tuple(spec.tile_args):
        raise ValueError(
            f"{spec.name}: HIP family tile args {desc['tile_args']} differ from the spec's "
            f"{list(spec.tile_args)}"
        )
    dims = [int(dim_sizes[d]) for d in spec.dim_vars]
    constraints = hip.manifest(spec.name, hw_variant, dims, dtype_code)
    names = spec.input_names()
    meta = {
        "kernel": spec.name,
        "hw_variant": hw_variant,
        "tile_variant": tile_variant,
        "dims": dims,
        "dim_vars": list(spec.dim_vars),
        "tile_args": list(spec.tile_args),
        "input_names": names,
        "input_shapes": [list(sh) for sh in spec.input_shapes(dim_sizes)],
        "target": target,
    }
    return _TEMPLATE.format(
        name=spec.name,
        i=hw_variant,
        j=tile_variant,
        summary=desc["summary"],
        dims=dict(zip(spec.dim_vars, dims)),
        fn=safe_name(spec.name),
        manifest_name=MANIFEST_NAME,
        manifest=manifest_literal(constraints),
        meta_name="__axon_hip_kernel__",
        meta=meta,
        params=", ".join([*names, *spec.tile_args]),
        inputs="".join(f"{n}, " for n in names),
        tiles="".join(f"{t}, " for t in spec.tile_args),
    )


def emit_variant_modules(spec: KernelSpec, dim_sizes: dict[str, int], paths: RunPaths,
                         dtype: Any | None = None, target: str = "gfx950") -> list[Path]:
    """Write every hw variant's module for these sizes; returns their paths.
    Raises LookupError when the registry has no family for the spec."""
    from enzyme_amd import hip

    n = hip.variant_count(spec.name)
    if n == 0:
        raise LookupError(f"no HIP variant set for kernel '{spec.name}'")
    code = input0_dtype_code(spec, dtype)
    fn = safe_name(spec.name)
    paths.run_dir.mkdir(parents=True, exist_ok=True)
    for stale in paths.run_dir.glob(f"{fn}__v*_t*.py"):
        stale.unlink()
    written = []
    for i in range(n):
        p = paths.variant_module(fn, i, 0)
        p.write_text(variant_module_text(spec, dim_sizes, i, 0, code, target))
        written.append(p)
    return written
