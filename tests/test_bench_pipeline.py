"""Host tests of the streaming compile -> bench pipeline and its durable
store, with in-process thread pools and stub workers (the reference's
tests/test_bench_resume.py strategy): every key gets exactly one terminal
row, interrupted runs keep exactly their fsynced rows and resume the rest,
torn tails are truncated, damaged stores refuse publication, artefact dirs
are bounded and reclaimed only after their row is durable."""

from __future__ import annotations

import csv
import dataclasses
import os
import threading
from collections import Counter
from concurrent.futures import ThreadPoolExecutor
from itertools import product

import pytest

from axon import bench_runner
from axon.bench_runner import BenchStats
from axon.paths import run_paths
from tests._specs import load_spec

DIMS = {"m": 16, "n": 64}


def spec_with(options=(1, 2)):
    return dataclasses.replace(load_spec("rmsnorm"), tile_options=options)


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    for var in ("AXON_KEEP_NEFF", "AXON_MAX_LIVE_NEFFS", "AXON_COMPILE_WORKERS", "HIP_VISIBLE_DEVICES"):
        monkeypatch.delenv(var, raising=False)


def _write_art(path: str) -> None:
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w") as f:
        f.write("{}")


def ok_compile(args):
    _write_art(args[5])
    return (args[2], args[5], None)


def ok_bench(args):
    return BenchStats(1.0, 1.0, 1.0, 1.0, 0.0, outputs=None)


def install(monkeypatch, compile_fn=ok_compile, bench_fn=ok_bench, *, compile_workers=2, devices=1):
    def pools(*, n_compile, core_specs):
        return ThreadPoolExecutor(n_compile), [ThreadPoolExecutor(1) for _ in core_specs]

    monkeypatch.setattr(bench_runner, "_make_pipeline_pools", pools)
    monkeypatch.setattr(bench_runner, "_visible_gpu_count", lambda: devices)
    monkeypatch.setattr(bench_runner, "_compile_one_variant", compile_fn)
    monkeypatch.setattr(bench_runner, "_bench_one_artifact", bench_fn)
    monkeypatch.setenv("AXON_COMPILE_WORKERS", str(compile_workers))


def bench(spec, paths, **kw):
    paths.run_dir.mkdir(parents=True, exist_ok=True)
    return bench_runner.run_hip_bench(
        spec, DIMS, hw_variant=0, tile_variant=kw.pop("tile_variant", 0),
        module_path=str(paths.variant_module("rmsnorm", 0, 0)), function_name="rmsnorm",
        warmup=1, bench=1, paths=paths, rtol=1e-2, atol=1e-2, **kw,
    )


def expected(options, tile_variant=0):
    return {("1", "lnc1", "0", str(tile_variant), str(a), str(b)) for a, b in product(options, repeat=2)}


def keys_of(spec, path):
    with open(path, newline="") as f:
        r = csv.DictReader(f)
        assert r.fieldnames == bench_runner.result_columns(spec)
        return [tuple(row[c] for c in bench_runner.key_columns(spec)) for row in r]


def rows_of(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def art_dirs(paths):
    return sorted(p.name for p in paths.run_dir.glob("__v*_tiles_*") if p.is_dir())


def record(spec, tiles):
    vals = {"m": 16, "n": 64, "lnc": 1, "sharding": "lnc1", "hw_variant": 0, "tile_variant": 0,
            "TILES_M": tiles[0], "TILES_N": tiles[1], "mean_ms": 1.0, "median_ms": 1.0, "min_ms": 1.0,
            "max_ms": 1.0, "std_dev_ms": 0.0, "correct": "", "max_abs_err": "", "error": "", "mode": ""}
    return ",".join(str(vals[c]) for c in bench_runner.result_columns(spec))


def test_column_layout():
    spec = spec_with()
    assert bench_runner.tile_cols(spec.tile_args) == ["TILES_M", "TILES_N"]
    assert bench_runner.key_columns(spec) == ["lnc", "sharding", "hw_variant", "tile_variant",
                                              "TILES_M", "TILES_N"]
    assert bench_runner.result_columns(spec) == [
        "m", "n", "lnc", "sharding", "hw_variant", "tile_variant", "TILES_M", "TILES_N", "mean_ms",
        "median_ms", "min_ms", "max_ms", "std_dev_ms", "correct", "max_abs_err", "error", "mode"]


def test_full_case_publishes_exactly_once_per_key(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with()
    paths = run_paths(spec, "out/rmsnorm_t.csv")
    install(monkeypatch)
    exp = set()
    for tv in (0, 1):
        got = bench(spec, paths, tile_variant=tv)
        assert got == expected(spec.tile_options, tv)
        exp |= got
    assert not paths.csv.exists()
    bench_runner.publish_results(spec, paths, exp)
    assert paths.csv.read_text() == paths.results.read_text()
    counts = Counter(keys_of(spec, paths.csv))
    assert set(counts) == exp and set(counts.values()) == {1}


def test_manifest_prunes_before_compile(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with()
    paths = run_paths(spec, "out/rmsnorm_f.csv")
    mod = paths.variant_module("rmsnorm", 0, 0)
    mod.parent.mkdir(parents=True)
    mod.write_text(
        "__axon_tile_constraints__ = {'version': 1, 'constraints': ("
        "{'tile_arg': 'TILES_IN_BLOCK_M', 'extent': 1, 'tile_size': 1, 'require_divisible': False},)}\n"
    )
    compiled = []

    def comp(args):
        compiled.append(args[2])
        return ok_compile(args)

    install(monkeypatch, comp)
    got = bench(spec, paths)
    assert got == {("1", "lnc1", "0", "0", "1", "1"), ("1", "lnc1", "0", "0", "1", "2")}
    assert sorted(compiled) == [(1, 1), (1, 2)]
    assert bench(spec, paths, candidate_filter=False) == expected(spec.tile_options)


def test_compile_and_bench_overlap(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with()
    paths = run_paths(spec, "out/rmsnorm_o.csv")
    monkeypatch.setenv("AXON_MAX_LIVE_NEFFS", "4")
    blocker = (1, 1)
    entered, other, release = threading.Event(), threading.Event(), threading.Event()

    def comp(args):
        if args[2] == blocker:
            entered.set()
            release.wait(30)
        return ok_compile(args)

    def ben(args):
        if args[2] != blocker:
            other.set()
        return ok_bench(args)

    install(monkeypatch, comp, ben, compile_workers=2)
    out = {}

    def referee():
        out["entered"] = entered.wait(30)
        out["overlap"] = other.wait(30)
        release.set()

    t = threading.Thread(target=referee)
    t.start()
    try:
        got = bench(spec, paths)
    finally:
        release.set()
        t.join(60)
    assert out.get("entered") and out.get("overlap")
    assert got == expected(spec.tile_options)


class _Stop(BaseException):
    pass


def interrupt_after(monkeypatch, k):
    real = bench_runner._append_result_row
    seen = {"n": 0}

    def wrapper(*a, **kw):
        if seen["n"] >= k:
            raise _Stop()
        real(*a, **kw)
        seen["n"] += 1

    monkeypatch.setattr(bench_runner, "_append_result_row", wrapper)


def test_interrupt_then_resume_runs_only_missing_keys(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with()
    paths = run_paths(spec, "out/rmsnorm_r.csv")
    with monkeypatch.context() as mp:
        install(mp, compile_workers=1)
        interrupt_after(mp, 2)
        with pytest.raises(_Stop):
            bench(spec, paths)
    text = paths.results.read_text()
    assert text.endswith("\n") and len(text.splitlines()) == 3
    assert not paths.csv.exists()
    done = bench_runner.read_result_keys(spec, paths.results)
    remaining = {k[-2:] for k in expected(spec.tile_options) - done}
    seen = []

    def comp(args):
        seen.append(tuple(str(v) for v in args[2]))
        return ok_compile(args)

    install(monkeypatch, comp)
    assert bench(spec, paths) == expected(spec.tile_options)
    assert set(seen) == remaining and len(seen) == len(remaining)
    counts = Counter(keys_of(spec, paths.results))
    assert set(counts.values()) == {1}


@pytest.mark.parametrize("mode", ["missing", "raises", "assert"])
def test_compile_failure_is_one_terminal_row(tmp_path, monkeypatch, mode):
    monkeypatch.chdir(tmp_path)
    spec = spec_with((1,))
    paths = run_paths(spec, f"out/rmsnorm_{mode}.csv")

    def comp(args):
        os.makedirs(os.path.dirname(args[5]), exist_ok=True)
        if mode == "raises":
            raise RuntimeError("compile blew up")
        return (args[2], None, "assert" if mode == "assert" else "artifact_missing")

    def ben(args):
        raise AssertionError("a failed compile must never reach the device")

    install(monkeypatch, comp, ben)
    assert bench(spec, paths) == expected((1,))
    rows = rows_of(paths.results)
    assert len(rows) == 1 and rows[0]["error"].startswith(("compile:", "RuntimeError"))
    assert not art_dirs(paths)


def test_bench_failure_is_one_terminal_row(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with((1,))
    paths = run_paths(spec, "out/rmsnorm_bf.csv")

    def ben(args):
        raise RuntimeError("device fell over")

    install(monkeypatch, ok_compile, ben)
    bench(spec, paths)
    rows = rows_of(paths.results)
    assert len(rows) == 1 and "device fell over" in rows[0]["error"]
    assert not art_dirs(paths)


def test_correctness_column_from_outputs(tmp_path, monkeypatch):
    """A device result is checked against the spec's torch_ref on the same
    seeded inputs: the exact answer is correct, a perturbed one is not, and
    max_abs_err records the gap."""
    import numpy as np

    from enzyme_amd.dtypes import to_f32_numpy
    from enzyme_amd.kernel_spec import SEED

    monkeypatch.chdir(tmp_path)
    spec = spec_with((1,))
    (x,) = spec.make_inputs(**DIMS, rng=np.random.default_rng(SEED))
    good = spec.baseline_op(to_f32_numpy(x))
    for label, out, want in (("good", good, "True"), ("bad", good + 0.5, "False")):
        paths = run_paths(spec, f"out/rmsnorm_{label}.csv")

        def ben(args, out=out):
            return BenchStats(1.0, 1.0, 1.0, 1.0, 0.0, outputs=(out,))

        install(monkeypatch, ok_compile, ben)
        bench(spec, paths)
        r = rows_of(paths.results)[0]
        assert r["correct"] == want
        assert (float(r["max_abs_err"]) > 0.4) == (label == "bad")


def test_correctness_decided_by_torch_ref_when_present(tmp_path, monkeypatch):
    """cumsum at 128 x 32768 on N(0,1) inputs: the exact prefix sums
    (torch.cumsum, double accumulation) are correct at the case tolerance
    1e-3, although the reference's numpy baseline_op (sequential fp32) is
    more than 1e-3 away from them; an output off the exact sums by 5e-3 is
    not correct."""
    import numpy as np
    import torch

    from enzyme_amd.kernel_spec import SEED

    monkeypatch.chdir(tmp_path)
    spec = dataclasses.replace(load_spec("cumsum"), tile_options=(1,))
    dims = {"m": 128, "n": 32768}
    (x,) = spec.make_inputs(**dims, rng=np.random.default_rng(SEED))
    exact = torch.cumsum(torch.as_tensor(x), dim=-1).numpy()
    assert np.abs(spec.baseline_op(x) - exact).max() > 1.5e-3
    for label, out, want in (("exact", exact, "True"), ("off", exact + 5e-3, "False")):
        paths = run_paths(spec, f"out/cumsum_{label}.csv")
        paths.run_dir.mkdir(parents=True, exist_ok=True)

        def ben(args, out=out):
            return BenchStats(1.0, 1.0, 1.0, 1.0, 0.0, outputs=(out,))

        install(monkeypatch, ok_compile, ben)
        bench_runner.run_hip_bench(
            spec, dims, hw_variant=0, tile_variant=0,
            module_path=str(paths.variant_module("cumsum", 0, 0)), function_name="cumsum",
            warmup=1, bench=1, paths=paths, rtol=1e-3, atol=1e-3, candidate_filter=False,
        )
        assert rows_of(paths.results)[0]["correct"] == want


def test_torn_tail_is_truncated_before_append(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with()
    paths = run_paths(spec, "out/rmsnorm_tt.csv")
    paths.run_dir.mkdir(parents=True)
    cols = ",".join(bench_runner.result_columns(spec))
    paths.results.write_text(cols + "\n" + record(spec, (1, 1)) + "\n" + record(spec, (1, 2))[:15])
    assert bench_runner.read_result_keys(spec, paths.results) == {("1", "lnc1", "0", "0", "1", "1")}
    assert paths.results.read_text().endswith("\n")
    install(monkeypatch)
    got = bench(spec, paths)
    counts = Counter(keys_of(spec, paths.results))
    assert set(counts) == got and set(counts.values()) == {1}


@pytest.mark.parametrize(("damage", "msg"), [("malformed", "malformed record"),
                                              ("duplicate", "duplicate key"), ("drift", "column drift")])
def test_damaged_store_stops_publication(tmp_path, monkeypatch, damage, msg):
    monkeypatch.chdir(tmp_path)
    spec = spec_with()
    paths = run_paths(spec, f"out/rmsnorm_{damage}.csv")
    paths.run_dir.mkdir(parents=True)
    cols = bench_runner.result_columns(spec)
    if damage == "malformed":
        lines = [",".join(cols), record(spec, (1, 1)), ",".join(record(spec, (1, 2)).split(",")[:-3])]
    elif damage == "duplicate":
        lines = [",".join(cols), record(spec, (1, 1)), record(spec, (1, 1))]
    else:
        lines = [",".join([*cols, "extra"]), record(spec, (1, 1)) + ",0"]
    paths.results.write_text("\n".join(lines) + "\n")
    with pytest.raises(AssertionError, match=msg):
        bench_runner.publish_results(spec, paths, expected(spec.tile_options))
    assert not paths.csv.exists()


def test_incomplete_coverage_stops_publication(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with()
    paths = run_paths(spec, "out/rmsnorm_cov.csv")
    install(monkeypatch)
    got = bench(spec, paths)
    with pytest.raises(AssertionError):
        bench_runner.publish_results(spec, paths, got | {("2", "lnc2", "0", "0", "1", "1")})
    with pytest.raises(AssertionError):
        bench_runner.publish_results(spec, paths, got - {next(iter(got))})
    assert not paths.csv.exists()


def test_stale_artifacts_cleared_and_keep_honoured(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with((1,))
    paths = run_paths(spec, "out/rmsnorm_st.csv")
    stale = paths.run_dir / "__v0_t0_tiles_9_9"
    stale.mkdir(parents=True)
    install(monkeypatch)
    bench(spec, paths)
    assert not stale.exists() and not art_dirs(paths)
    monkeypatch.setenv("AXON_KEEP_NEFF", "1")
    paths2 = run_paths(spec, "out/rmsnorm_keep.csv")
    bench(spec, paths2)
    assert art_dirs(paths2) == ["__v0_t0_tiles_1_1"]


def test_live_artifacts_bounded(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with((1, 2, 4, 8))
    paths = run_paths(spec, "out/rmsnorm_live.csv")
    monkeypatch.setenv("AXON_MAX_LIVE_NEFFS", "2")
    peak = {"n": 0}
    lock = threading.Lock()

    def comp(args):
        r = ok_compile(args)
        with lock:
            peak["n"] = max(peak["n"], len(art_dirs(paths)))
        return r

    install(monkeypatch, comp, compile_workers=4, devices=2)
    bench(spec, paths)
    assert peak["n"] <= 2
    assert len(keys_of(spec, paths.results)) == 16


def test_lnc2_is_recorded_as_skipped(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    spec = spec_with((1,))
    paths = run_paths(spec, "out/rmsnorm_l2.csv")
    install(monkeypatch)
    got = bench(spec, paths, lnc=2, sharding="shard_P")
    rows = rows_of(paths.results)
    assert len(rows) == 1 and "multi-device" in rows[0]["error"] and len(got) == 1
