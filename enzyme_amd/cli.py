"""`axon <kernel-path> --sizes N... [flags]` for the HIP backend.

Same command surface as src/axon/cli.py:825-1129 of the reference: a spec
is loaded by path (:100-135), `--sizes` binds positionally to `dim_vars` and
a wrong count exits 2 (:1044-1051), `--rtol` and `--atol` together mark a
head-to-head case whose id is the `--out` stem minus `<kernel>_`
(:1067-1081), and `--phase emit|bench|all` splits the run (:491-523):

* emit  writes one variant module per hw variant of the spec's HIP family
        (the registry in libaxon_hip.so replaces synthesis + NKI emission);
* bench discovers `<fn>__v*_t*.py` in the run dir and benches each on the GPU,
        exiting 2 when there are none (:307-354);
* all   does both.

The synthesis knobs (--synthesis-timeout-seconds, --synth-workers,
--tensor-rounds, --isa-rounds, --max-hw-graphs, --from-cache, --cache-dir)
are accepted so existing Makefiles run unchanged; there is no synthesis
here, so they change nothing. `--lnc 2` is refused: multi-device sharding is
not part of this backend.
"""

from __future__ import annotations

import argparse
import importlib.util
import inspect
import math
import sys
from pathlib import Path
from typing import Any

import numpy as np

from enzyme_amd import dtypes as _dt
from enzyme_amd.bench_runner import (
    DEFAULT_TARGET,
    ResultKey,
    clear_stale_artifacts,
    publish_results,
    run_baseline,
    run_hip_bench,
)
from enzyme_amd.emit import emit_variant_modules, safe_name
from enzyme_amd.kernel_spec import KernelSpec
from enzyme_amd.paths import RunPaths, run_paths
from enzyme_amd.winner import export_winner, pick_winner

DTYPE_CHOICES: tuple[str, ...] = ("bfloat16", "float16", "float32")

_DEFAULT_RTOL = 2e-2
_DEFAULT_ATOL = 2e-2
_DEFAULT_CACHE_DIR = "cache"
_DEFAULT_SATURATION_ROUNDS = 50
DEFAULT_SYNTHESIS_WALL_CLOCK_SECONDS = 3600.0
DEFAULT_MAX_HW_GRAPHS = 256

# Tests and callers patch this name, as in the reference.
run_nki_bench = run_hip_bench


def _positive_int(value: str) -> int:
    v = int(value)
    if v <= 0:
        raise argparse.ArgumentTypeError("must be greater than zero")
    return v


def _nonnegative_int(value: str) -> int:
    v = int(value)
    if v < 0:
        raise argparse.ArgumentTypeError("must not be negative")
    return v


def _positive_finite_float(value: str) -> float:
    v = float(value)
    if not math.isfinite(v) or v <= 0:
        raise argparse.ArgumentTypeError("must be a finite value greater than zero")
    return v


def _spec_default_dtype_name(spec: KernelSpec) -> str:
    param = inspect.signature(spec.make_inputs).parameters.get("dtype")
    if param is None or param.default is inspect.Parameter.empty:
        return "float32"
    return _dt.dtype_name(param.default)


def _load_spec(path: str) -> KernelSpec:
    """Load `SPEC` from a spec package directory or a single-file spec."""
    p = Path(path).expanduser().resolve()
    search = None
    if p.is_dir():
        init = p / "__init__.py"
        if not init.is_file():
            print(f"kernel-spec dir has no __init__.py: {p}", file=sys.stderr)
            sys.exit(2)
        search = [str(p)]
        module_name = f"_axon_kernel_spec_{safe_name(p.name)}"
        target = init
    elif p.is_file():
        module_name = f"_axon_kernel_spec_{safe_name(p.stem)}"
        target = p
    else:
        print(f"kernel-spec file not found: {p}", file=sys.stderr)
        sys.exit(2)
    spec = importlib.util.spec_from_file_location(module_name, target, submodule_search_locations=search)
    if spec is None or spec.loader is None:
        print(f"could not load kernel-spec from {p}", file=sys.stderr)
        sys.exit(2)
    module = importlib.util.module_from_spec(spec)
    sys.modules[module_name] = module
    spec.loader.exec_module(module)
    obj = getattr(module, "SPEC", None)
    if not isinstance(obj, KernelSpec):
        print(f"{p} does not define a top-level `SPEC: KernelSpec`", file=sys.stderr)
        sys.exit(2)
    return obj


def _bench_existing_modules(
    spec: KernelSpec,
    dim_sizes: dict[str, int],
    paths: RunPaths,
    function_name: str,
    *,
    warmup: int,
    bench: int,
    target: str | None,
    dtype: Any | None,
    rtol: float,
    atol: float,
    candidate_filter: bool,
    candidate_budget: int,
) -> set[ResultKey]:
    modules = sorted(paths.run_dir.glob(f"{function_name}__v*_t*.py"))
    if not modules:
        print(
            f"--phase bench: no emitted variant modules under {paths.run_dir}; "
            f"run --phase emit first",
            file=sys.stderr,
        )
        sys.exit(2)
    paths.csv.unlink(missing_ok=True)
    expected: set[ResultKey] = set()
    for module in modules:
        i_s, j_s = module.stem.rsplit("__v", 1)[1].split("_t", 1)
        expected |= run_nki_bench(
            spec,
            dim_sizes,
            hw_variant=int(i_s),
            tile_variant=int(j_s),
            module_path=str(module),
            function_name=function_name,
            warmup=warmup,
            bench=bench,
            target=target,
            dtype=dtype,
            paths=paths,
            rtol=rtol,
            atol=atol,
            candidate_filter=candidate_filter,
            candidate_budget=candidate_budget,
        )
    return expected


def _finish_run(
    spec: KernelSpec,
    paths: RunPaths,
    *,
    pick_by: str,
    rtol: float,
    atol: float,
    kernel_path: str | None,
    case_id: str | None,
    case_dtype: str | None,
) -> None:
    winner = pick_winner(paths.csv, spec, pick_by, rtol=rtol, atol=atol)  # type: ignore[arg-type]
    assert winner is not None, f"{spec.name}: no timed variants in {paths.csv}"
    print(
        f"\nwinner: v{winner.hw_variant}_t{winner.tile_variant} tiles {winner.tile_values} "
        f"median {winner.median_ms} ms"
    )
    if case_id is not None:
        if spec.torch_ref is None:
            raise ValueError(f"head-to-head case {spec.name}_{case_id} requires spec.torch_ref")
        if kernel_path is None or case_dtype is None:
            raise ValueError("head-to-head export needs kernel_path and case_dtype")
        export_winner(
            spec, winner, case_id=case_id, kernel_path=kernel_path, paths=paths,
            dtype=case_dtype, rtol=rtol, atol=atol,
        )


def _publish_and_finish(
    spec: KernelSpec,
    paths: RunPaths,
    expected: set[ResultKey],
    *,
    pick_by: str,
    rtol: float,
    atol: float,
    kernel_path: str | None,
    case_id: str | None,
    case_dtype: str | None,
) -> None:
    publish_results(spec, paths, expected)
    clear_stale_artifacts(paths)
    _finish_run(
        spec, paths, pick_by=pick_by, rtol=rtol, atol=atol, kernel_path=kernel_path,
        case_id=case_id, case_dtype=case_dtype,
    )


def trace_kernel(
    spec: KernelSpec,
    dim_sizes: dict[str, int],
    *,
    warmup: int,
    bench: int,
    target: str | None = None,
    dtype: Any | None = None,
    out: str | None = None,
    rtol: float = _DEFAULT_RTOL,
    atol: float = _DEFAULT_ATOL,
    kernel_path: str | None = None,
    case_id: str | None = None,
    case_dtype: str | None = None,
    pick_by: str = "median",
    lnc: int = 1,
    phase: str = "all",
    candidate_filter: bool = True,
    candidate_budget: int = 8,
    **_synthesis_knobs: Any,
) -> int | None:
    """Emit, bench, or both for one spec at one size binding."""
    print("\n" + "=" * 80)
    print(f"Tracing kernel: {spec.name} (phase={phase})")
    print("=" * 80)
    if lnc >= 2:
        print("--lnc 2: multi-device sharding is not part of this backend", file=sys.stderr)
        sys.exit(2)
    paths = run_paths(spec, out)
    fn = safe_name(spec.name)
    if phase in ("emit", "all"):
        try:
            written = emit_variant_modules(spec, dim_sizes, paths, dtype=dtype, target=target or DEFAULT_TARGET)
        except LookupError as e:
            print(str(e), file=sys.stderr)
            return 2
        paths.csv.unlink(missing_ok=True)
        print(f"--- {spec.name} :: wrote {len(written)} HIP variant module(s) under {paths.run_dir}")
        if phase == "emit":
            print(
                f"\n--phase emit done: {len(written)} variant module(s) under {paths.run_dir}. "
                "Bench them on a GPU with the same case args plus --phase bench."
            )
            return None
    expected = _bench_existing_modules(
        spec, dim_sizes, paths, fn, warmup=warmup, bench=bench, target=target, dtype=dtype,
        rtol=rtol, atol=atol, candidate_filter=candidate_filter, candidate_budget=candidate_budget,
    )
    _publish_and_finish(
        spec, paths, expected, pick_by=pick_by, rtol=rtol, atol=atol, kernel_path=kernel_path,
        case_id=case_id, case_dtype=case_dtype,
    )
    return None


def _build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description="Bench the HIP variant set of a kernel spec on a GPU.")
    p.add_argument("kernel", help="Path to a kernel-spec package dir or .py file with a top-level SPEC.")
    p.add_argument(
        "--sizes", type=int, nargs="+", required=True, metavar="N",
        help="Concrete sizes, bound positionally to the spec's dim_vars.",
    )
    p.add_argument("--target", default=DEFAULT_TARGET, help="GPU target (gfx950).")
    p.add_argument("--dtype", choices=DTYPE_CHOICES, default=None,
                   help="Override the input dtype of the spec's make_inputs.")
    p.add_argument("--out", default=None, metavar="PATH",
                   help="Run stem: out/<stem>.csv is the case CSV, out/<stem>/ the run dir.")
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--bench", type=int, default=100)
    p.add_argument("--synthesis-timeout-seconds", type=_positive_finite_float,
                   default=DEFAULT_SYNTHESIS_WALL_CLOCK_SECONDS, metavar="SECONDS",
                   help="Accepted for compatibility; there is no synthesis.")
    p.add_argument("--mode", choices=("variants", "baseline", "both"), default="variants",
                   help="'variants' (HIP), 'baseline' (spec torch_ref on the host CPU), or both.")
    p.add_argument("--pick-by", choices=("median", "mean", "min"), default="median")
    p.add_argument("--phase", choices=("emit", "bench", "all"), default="all")
    p.add_argument("--lnc", type=int, choices=(1, 2), default=1)
    p.add_argument("--synth-workers", dest="synth_workers", type=_positive_int, default=None,
                   metavar="N", help="Accepted for compatibility; there is no synthesis.")
    p.add_argument("--max-hw-graphs", dest="max_hw_graphs", type=_nonnegative_int,
                   default=DEFAULT_MAX_HW_GRAPHS, metavar="N",
                   help="Accepted for compatibility; there is no synthesis.")
    p.add_argument("--candidate-filter", action=argparse.BooleanOptionalAction, default=True,
                   help="Apply the variant's tile manifest before compiling (default on).")
    p.add_argument("--candidate-budget", type=_nonnegative_int, default=8, metavar="N",
                   help="Legal tile tuples kept per variant (0 = all).")
    p.add_argument("--tensor-rounds", dest="tensor_rounds", type=_positive_int,
                   default=_DEFAULT_SATURATION_ROUNDS, metavar="N")
    p.add_argument("--isa-rounds", dest="isa_rounds", type=_positive_int,
                   default=_DEFAULT_SATURATION_ROUNDS, metavar="N")
    p.add_argument("--from-cache", dest="from_cache", action="store_true")
    p.add_argument("--cache-dir", dest="cache_dir", default=_DEFAULT_CACHE_DIR, metavar="PATH")
    p.add_argument("--rtol", type=float, default=None,
                   help="With --atol, marks a head-to-head case (winner + harness exported).")
    p.add_argument("--atol", type=float, default=None)
    return p


def _run(args: argparse.Namespace) -> int:
    spec = _load_spec(args.kernel)
    if len(args.sizes) != len(spec.dim_vars):
        print(
            f"{spec.name}: --sizes expects {len(spec.dim_vars)} values for dims "
            f"{list(spec.dim_vars)} in order, got {len(args.sizes)}",
            file=sys.stderr,
        )
        sys.exit(2)
    dim_sizes = dict(zip(spec.dim_vars, args.sizes, strict=True))
    if args.from_cache and args.phase == "bench":
        print("--from-cache does not apply to --phase bench", file=sys.stderr)
        sys.exit(2)
    paths = run_paths(spec, args.out)
    dtype = _dt.resolve(args.dtype) if args.dtype else None
    rtol = args.rtol if args.rtol is not None else _DEFAULT_RTOL
    atol = args.atol if args.atol is not None else _DEFAULT_ATOL
    case_id = case_dtype = None
    status = 0
    if args.rtol is not None and args.atol is not None:
        prefix = f"{spec.name}_"
        if not paths.csv.stem.startswith(prefix):
            print(
                f"{spec.name}: head-to-head run needs an --out stem of the form "
                f"'{spec.name}_<case_id>.csv', got {paths.csv.stem!r}",
                file=sys.stderr,
            )
            sys.exit(2)
        case_id = paths.csv.stem[len(prefix):]
        case_dtype = args.dtype or _spec_default_dtype_name(spec)
    if args.mode in ("variants", "both"):
        rc = trace_kernel(
            spec,
            dim_sizes,
            warmup=args.warmup,
            bench=args.bench,
            target=args.target,
            dtype=dtype,
            out=args.out,
            rtol=rtol,
            atol=atol,
            kernel_path=str(Path(args.kernel).expanduser().resolve()),
            case_id=case_id,
            case_dtype=case_dtype,
            pick_by=args.pick_by,
            lnc=args.lnc,
            phase=args.phase,
            synthesis_timeout_seconds=args.synthesis_timeout_seconds,
            synth_workers=args.synth_workers,
            tensor_rounds=args.tensor_rounds,
            isa_rounds=args.isa_rounds,
            cache_dir=args.cache_dir,
            from_cache=args.from_cache,
            max_hw_graphs=args.max_hw_graphs or None,
            candidate_filter=args.candidate_filter,
            candidate_budget=args.candidate_budget,
        )
        if rc is not None:
            status = rc
    if args.mode in ("baseline", "both"):
        if spec.baseline_op is None and spec.torch_ref is None:
            print(f"kernel '{spec.name}' has no baseline_op set", file=sys.stderr)
            return 2
        paths.baseline_csv.unlink(missing_ok=True)
        run_baseline(spec, dim_sizes, warmup=args.warmup, bench=args.bench, target=args.target,
                     dtype=dtype, paths=paths)
    return status


def main(argv: list[str] | None = None) -> None:
    args = _build_parser().parse_args(argv)
    sys.exit(_run(args))


if __name__ == "__main__":
    main()
