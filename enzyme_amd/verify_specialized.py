"""Check that a specialized winner is equivalent to the parameterized one.

The contract of the reference's tools/verify_specialized.py (docstring 1-30):
`specialize_winner` moves the winning `TILES_IN_BLOCK_*` values from the
signature into constants, so both modules must build the same kernel, give
the same outputs and run at the same speed. For one case this tool

  1. resolves each module to the launch it performs (the kernel family, hw
     variant, tile tuple, dims and input shapes it hands to libaxon_hip.so),
     with the parameterized winner called with the case's tile values and
     the specialized one with none, and compares the two launch plans (this
     backend's artefact: the instantiation is selected from an ahead-of-time
     table, so an identical plan is an identical kernel binary);
  2. checks the plan against the library (`axon_variant_check`);
  3. on a GPU, runs both modules on the case's seeded inputs and compares
     each output with the spec's fp32 `torch_ref` at the case tolerance, and
     the two modules' outputs with each other bit for bit;
  4. benchmarks both launches (HIP events per launch, rotating buffer sets)
     and prints the medians.

Both modules are loaded under the same module name, one after the other, as
the reference does (reference lines 19-25). The launch plan is read by
calling the module's entry with a recorder in place of its `_hip` binding,
so the module's own code decides what it launches.

    python -m enzyme_amd.verify_specialized rmsnorm_h1024 [--runs-dir out]
        [--specialized-dir winners] [--bench 50] [--no-device]

Exit status: 0 equivalent, 1 not equivalent (or a device check failed),
2 missing files or a malformed module.
"""

from __future__ import annotations

import argparse
import hashlib
import importlib.util
import json
import math
import statistics
import sys
from dataclasses import dataclass, field
from pathlib import Path

from enzyme_amd.specialize_winner import REPO, TILE_PREFIX, SpecializeError, read_case

MODULE_NAME = "_axon_verify_kernel"  # identical for both arms, on purpose


class VerifyError(RuntimeError):
    """A file is missing or a module cannot be resolved to a launch."""


@dataclass
class Report:
    stem: str
    plan_param: dict
    plan_spec: dict
    legal: bool | None = None
    legal_why: str = ""
    device: bool = False
    correct_param: bool | None = None
    correct_spec: bool | None = None
    bit_identical: bool | None = None
    max_abs_err: float | None = None
    median_us_param: float | None = None
    median_us_spec: float | None = None
    notes: list[str] = field(default_factory=list)

    @property
    def same_plan(self) -> bool:
        return plan_digest(self.plan_param) == plan_digest(self.plan_spec)

    @property
    def ok(self) -> bool:
        checks = [self.same_plan, self.legal is not False]
        if self.device:
            checks += [bool(self.correct_param), bool(self.correct_spec), bool(self.bit_identical)]
        return all(checks)


def plan_digest(plan: dict) -> str:
    return hashlib.sha256(json.dumps(plan, sort_keys=True).encode()).hexdigest()[:16]


def _load(path: Path):
    if not path.is_file():
        raise VerifyError(f"{path} not found")
    sys.modules.pop(MODULE_NAME, None)
    spec = importlib.util.spec_from_file_location(MODULE_NAME, path)
    if spec is None or spec.loader is None:
        raise VerifyError(f"cannot import {path}")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[MODULE_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


class _Recorder:
    """Stands in for the module's `_hip`: records the launch instead of running it."""

    def __init__(self):
        self.calls = []

    def run_variant(self, meta, inputs, tiles):
        self.calls.append((dict(meta), [int(t) for t in tiles], len(list(inputs))))
        return None


def launch_plan(path: Path, entry: str, tiles: dict[str, int] | None) -> dict:
    """The launch the module's `entry` performs, called with placeholder
    inputs and (for the parameterized module) the case's tile values."""
    mod = _load(path)
    fn = getattr(mod, entry, None)
    if fn is None:
        raise VerifyError(f"{path.name}: no entry `{entry}`")
    meta = getattr(mod, "__axon_hip_kernel__", None)
    if not isinstance(meta, dict):
        raise VerifyError(f"{path.name}: no __axon_hip_kernel__ record")
    rec = _Recorder()
    real = getattr(mod, "_hip", None)
    mod._hip = rec
    try:
        fn(*([None] * len(meta["input_names"])), **(tiles or {}))
    except TypeError as exc:
        raise VerifyError(f"{path.name}: {entry} does not take the expected arguments ({exc})") from exc
    finally:
        mod._hip = real
        sys.modules.pop(MODULE_NAME, None)
    if len(rec.calls) != 1:
        raise VerifyError(f"{path.name}: {entry} made {len(rec.calls)} launches, expected 1")
    m, t, n_in = rec.calls[0]
    return {"kernel": m["kernel"], "hw_variant": int(m["hw_variant"]), "tiles": t,
            "dims": [int(d) for d in m["dims"]], "input_shapes": [list(s) for s in m.get("input_shapes", [])],
            "n_inputs": n_in, "target": m.get("target", "")}


def case_tiles(case: dict) -> dict[str, int]:
    return {k: int(v) for k, v in case["shape_args"].items() if k.startswith(TILE_PREFIX)}


def _spec_for(kernel: str):
    from enzyme_amd.cli import _load_spec

    path = REPO / "kernels" / kernel
    if not (path / "__init__.py").is_file():
        raise VerifyError(f"no spec package kernels/{kernel}")
    return _load_spec(str(path))


def _device_checks(report: Report, case: dict, param_path: Path, spec_path: Path, entry: str,
                   bench: int) -> None:
    import numpy as np
    import torch

    from enzyme_amd import dtypes as dt
    from enzyme_amd import hip
    from enzyme_amd.kernel_spec import SEED

    plan = report.plan_param
    spec = _spec_for(plan["kernel"])
    dims = {d: int(case["shape_args"][d]) for d in spec.dim_vars}
    host = spec.make_inputs(**dims, dtype=dt.resolve(case.get("dtype")), rng=np.random.default_rng(SEED))
    dev = [dt.to_torch(a).cuda() for a in host]
    _check_legal(report, [hip.dtype_code(t) for t in dev])
    with torch.no_grad():
        ref = spec.torch_ref(*[dt.to_f32_torch(a) for a in host])
    ref = ref if isinstance(ref, tuple) else (ref,)
    rtol, atol = float(case.get("rtol", 1e-2)), float(case.get("atol", 1e-2))

    outs = {}
    for arm, path, tiles in (("param", param_path, case_tiles(case)), ("spec", spec_path, None)):
        mod = _load(path)
        got = getattr(mod, entry)(*dev, **(tiles or {}))
        torch.cuda.synchronize()
        got = got if isinstance(got, tuple) else (got,)
        outs[arm] = [g.detach().float().cpu() for g in got]
        sys.modules.pop(MODULE_NAME, None)
    errs = []
    for arm in ("param", "spec"):
        ok = len(outs[arm]) == len(ref)
        for g, r in zip(outs[arm], ref):
            r = r.float().cpu()
            ok = ok and g.shape == r.shape and bool(torch.allclose(g, r, rtol=rtol, atol=atol))
            errs.append(float((g - r).abs().max()) if g.shape == r.shape and g.numel() else 0.0)
        setattr(report, f"correct_{arm}", ok)
    report.max_abs_err = max(errs) if errs else 0.0
    report.bit_identical = len(outs["param"]) == len(outs["spec"]) and all(
        torch.equal(a, b) for a, b in zip(outs["param"], outs["spec"]))

    if bench > 0:
        for arm, p in (("param", report.plan_param), ("spec", report.plan_spec)):
            ln = hip.Launcher(p["kernel"], p["hw_variant"], p["tiles"], p["dims"], dev)
            per_set = sum(t.numel() * t.element_size() for t in dev + ln.outputs)
            n_sets = max(1, min(16, math.ceil((256 << 20) / max(per_set, 1))))
            sets = [(dev, ln.outputs)] + [([t.clone() for t in dev], [torch.empty_like(o) for o in ln.outputs])
                                          for _ in range(n_sets - 1)]
            for i in range(max(10, bench)):
                ln.rebind(*sets[i % n_sets])
                ln.launch()
            torch.cuda.synchronize()
            times = []
            for i in range(bench):
                ln.rebind(*sets[i % n_sets])
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                ln.launch()
                b.record()
                times.append((a, b))
            torch.cuda.synchronize()
            setattr(report, f"median_us_{arm}", statistics.median(a.elapsed_time(b) * 1e3 for a, b in times))


def verify(stem: str, runs: Path, specialized: Path, bench: int = 50, device: bool | None = None) -> Report:
    """Compare the parameterized winner `<runs>/winners/<stem>.py` (tiles
    from `<stem>_case.py`) with the specialized `<specialized>/<stem>.py`."""
    source = runs / "winners"
    case_path = source / f"{stem}_case.py"
    if not case_path.is_file():
        raise VerifyError(f"{case_path} not found (is {stem} a head-to-head case?)")
    try:
        case = read_case(case_path)
    except SpecializeError as exc:
        raise VerifyError(str(exc)) from exc
    entry = case["entry_point"]
    param_path = source / case.get("kernel_rel", f"{stem}.py")
    spec_path = specialized / f"{stem}.py"
    tiles = case_tiles(case)
    if not tiles:
        raise VerifyError(f"{case_path.name}: the case binds no {TILE_PREFIX}* argument")
    report = Report(stem, launch_plan(param_path, entry, tiles), launch_plan(spec_path, entry, None))

    if device is None:
        try:
            import torch

            device = torch.cuda.is_available()
        except ImportError:
            device = False
    report.device = bool(device) and report.same_plan
    if report.device:
        _device_checks(report, case, param_path, spec_path, entry, bench)
    else:
        if device:
            report.notes.append("plans differ: device checks skipped")
        try:
            _check_legal(report, _input_codes(case, report.plan_param))
        except Exception as exc:  # noqa: BLE001 - reported, never fatal
            report.notes.append(f"legality not checked: {exc}")
    return report


def _check_legal(report: Report, codes: list[int]) -> None:
    from enzyme_amd import hip

    p = report.plan_param
    status, why = hip.check(p["kernel"], p["hw_variant"], p["tiles"], p["dims"], codes)
    report.legal, report.legal_why = status == hip.AXON_OK, why


def _input_codes(case: dict, plan: dict) -> list[int]:
    """Element types of the inputs the case builds (its spec's make_inputs,
    drawn at a tiny size: only the dtypes are used)."""
    import numpy as np

    from enzyme_amd import dtypes as dt
    from enzyme_amd import hip

    spec = _spec_for(plan["kernel"])
    dims = {d: 2 for d in spec.dim_vars}
    small = spec.make_inputs(**dims, dtype=dt.resolve(case.get("dtype")), rng=np.random.default_rng(0))
    return [hip.dtype_code(dt.to_torch(a)) for a in small]


def format_report(r: Report) -> str:
    lines = [f"{r.stem}:",
             f"  plan (parameterized) {plan_digest(r.plan_param)}  {json.dumps(r.plan_param, sort_keys=True)}",
             f"  plan (specialized)   {plan_digest(r.plan_spec)}  "
             + ("identical" if r.same_plan else json.dumps(r.plan_spec, sort_keys=True))]
    if r.legal is not None:
        lines.append(f"  library check        {'legal' if r.legal else 'REFUSED: ' + r.legal_why}")
    if r.device:
        lines.append(f"  fp32 torch_ref       parameterized {'ok' if r.correct_param else 'FAIL'}, "
                     f"specialized {'ok' if r.correct_spec else 'FAIL'} (max abs err {r.max_abs_err:.3g})")
        lines.append(f"  outputs              {'bit-identical' if r.bit_identical else 'DIFFER'}")
        if r.median_us_param is not None:
            lines.append(f"  median               parameterized {r.median_us_param:.2f} us, "
                         f"specialized {r.median_us_spec:.2f} us")
    lines += [f"  note: {n}" for n in r.notes]
    lines.append(f"  {'EQUIVALENT' if r.ok else 'NOT EQUIVALENT'}")
    return "\n".join(lines)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("stem", help="case stem, e.g. rmsnorm_h1024")
    ap.add_argument("--runs-dir", type=Path, default=Path.cwd() / "out",
                    help="run directory holding winners/<stem>.py and <stem>_case.py (default ./out)")
    ap.add_argument("--specialized-dir", type=Path, default=REPO / "winners",
                    help="where the specialized module is (default: the tracked winners/)")
    ap.add_argument("--bench", type=int, default=50, help="timed launches per arm (0: no benchmark)")
    ap.add_argument("--no-device", action="store_true", help="compare the launch plans only")
    a = ap.parse_args(argv)
    try:
        r = verify(a.stem, a.runs_dir.resolve(), a.specialized_dir.resolve(), a.bench,
                   device=False if a.no_device else None)
    except VerifyError as exc:
        print(f"error: {exc}", file=sys.stderr)
        return 2
    print(format_report(r))
    return 0 if r.ok else 1


if __name__ == "__main__":
    sys.exit(main())
