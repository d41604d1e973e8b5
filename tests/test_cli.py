"""`axon <kernel> --sizes ...` surface (src/axon/cli.py of the reference):
positional binding to dim_vars, exit codes, case ids, paths, and the
emit/bench phase split of this backend."""

from pathlib import Path
from types import SimpleNamespace

import pytest

from axon import cli
from axon.candidate_filter import read_manifest
from axon.paths import out_dir, run_paths
from tests._specs import KERNELS


def run_capture(monkeypatch, argv, spec):
    seen = {}
    monkeypatch.setattr(cli, "_load_spec", lambda p: spec)
    monkeypatch.setattr(cli, "trace_kernel", lambda s, d, **kw: seen.update(dims=d, **kw))
    with pytest.raises(SystemExit) as e:
        cli.main(argv)
    return e.value.code, seen


STUB = SimpleNamespace(name="stub", dim_vars=("m", "k", "n"))


@pytest.mark.parametrize(("sizes", "want"), [(["1024", "16384", "512"], {"m": 1024, "k": 16384, "n": 512}),
                                             (["8", "8", "8"], {"m": 8, "k": 8, "n": 8})])
def test_sizes_bind_positionally(monkeypatch, sizes, want):
    code, seen = run_capture(monkeypatch, ["stub", "--sizes", *sizes], STUB)
    assert code == 0 and seen["dims"] == want


@pytest.mark.parametrize("sizes", [["1", "2"], ["1", "2", "3", "4"], ["1", "x", "3"], ["m=1", "k=2", "n=3"]])
def test_bad_sizes_exit_2(monkeypatch, sizes):
    monkeypatch.setattr(cli, "_load_spec", lambda p: STUB)
    with pytest.raises(SystemExit) as e:
        cli.main(["stub", "--sizes", *sizes])
    assert e.value.code == 2


def test_head_to_head_case_id_and_dtype(monkeypatch):
    def mk(*, m, n, dtype="float32", rng):
        return ()

    spec = SimpleNamespace(name="mul", dim_vars=("m", "n"), make_inputs=mk)
    code, seen = run_capture(monkeypatch, ["mul", "--sizes", "4", "4", "--rtol", "1e-3", "--atol", "1e-3",
                                           "--out", "out/mul_bw_4k.csv"], spec)
    assert code == 0 and seen["case_id"] == "bw_4k" and seen["case_dtype"] == "float32"


def test_head_to_head_needs_kernel_prefixed_stem(monkeypatch):
    spec = SimpleNamespace(name="mul", dim_vars=("m", "n"), make_inputs=lambda **k: ())
    monkeypatch.setattr(cli, "_load_spec", lambda p: spec)
    with pytest.raises(SystemExit) as e:
        cli.main(["mul", "--sizes", "4", "4", "--rtol", "1", "--atol", "1", "--out", "out/other.csv"])
    assert e.value.code == 2


def test_bench_only_run_has_no_case(monkeypatch):
    code, seen = run_capture(monkeypatch, ["stub", "--sizes", "1", "2", "3", "--out", "out/x.csv"], STUB)
    assert code == 0 and seen["case_id"] is None and seen["case_dtype"] is None


def test_synthesis_knobs_accepted_and_validated(monkeypatch):
    code, seen = run_capture(monkeypatch, ["stub", "--sizes", "1", "2", "3", "--synth-workers", "4",
                                           "--synthesis-timeout-seconds", "7200"], STUB)
    assert code == 0 and seen["synth_workers"] == 4 and seen["synthesis_timeout_seconds"] == 7200.0
    monkeypatch.setattr(cli, "_load_spec", lambda p: STUB)
    for bad in (["--synth-workers", "0"], ["--synthesis-timeout-seconds", "inf"]):
        with pytest.raises(SystemExit) as e:
            cli.main(["stub", "--sizes", "1", "2", "3", *bad])
        assert e.value.code == 2


def test_run_paths_rules():
    spec = SimpleNamespace(name="mul")
    p = run_paths(spec, "out/mul_bw_4k.csv")
    base = Path("out/mul_bw_4k.csv").resolve()
    assert p.csv == base and p.run_dir == base.with_suffix("")
    assert p.variant_module("fn", 0, 2) == base.with_suffix("") / "fn__v0_t2.py"
    assert p.neff(0, 2, (1, 4)) == base.with_suffix("") / "__v0_t2_tiles_1_4" / "kernel.neff"
    assert p.artifact(0, 2, (1, 4)).parent == p.neff(0, 2, (1, 4)).parent
    assert p.baseline_csv == base.parent / "baseline_mul_bw_4k.csv"
    assert run_paths(spec, "out/foo") == run_paths(spec, "out/foo.csv")
    assert run_paths(spec, None).csv == (out_dir() / "nki_mul.csv").resolve()
    c = run_paths(spec, "results/")
    assert c.csv.name == "nki_mul.csv" and c.csv.parent.name == "results"


def test_load_spec_errors(tmp_path):
    for target in (tmp_path / "missing", tmp_path):
        with pytest.raises(SystemExit) as e:
            cli._load_spec(str(target))
        assert e.value.code == 2


def test_phase_emit_writes_hip_variant_modules(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)

    def boom(*a, **k):
        raise AssertionError("--phase emit must not bench")

    monkeypatch.setattr(cli, "run_nki_bench", boom)
    with pytest.raises(SystemExit) as e:
        cli.main([str(KERNELS / "cumsum_probs"), "--sizes", "64", "128256", "--phase", "emit",
                  "--out", "out/cumsum_probs_cfg"])
    assert e.value.code == 0
    mods = sorted((tmp_path / "out" / "cumsum_probs_cfg").glob("cumsum_probs__v*_t*.py"))
    assert [m.name for m in mods] == [f"cumsum_probs__v{i}_t0.py" for i in range(3)]
    cons = read_manifest(mods[1])
    assert {c.tile_arg for c in cons} == {"TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"}
    src = mods[0].read_text()
    assert "def cumsum_probs(probs, TILES_IN_BLOCK_M, TILES_IN_BLOCK_N):" in src


def test_phase_bench_without_modules_exits_2(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    with pytest.raises(SystemExit) as e:
        cli.main([str(KERNELS / "rmsnorm"), "--sizes", "8", "64", "--phase", "bench", "--out", "out/r"])
    assert e.value.code == 2


def test_lnc2_refused(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    with pytest.raises(SystemExit) as e:
        cli.main([str(KERNELS / "rmsnorm"), "--sizes", "8", "64", "--lnc", "2", "--out", "out/r"])
    assert e.value.code == 2


def test_phase_all_drives_emit_bench_publish_and_export(tmp_path, monkeypatch):
    """The full CLI flow with the device worker stubbed: emitted modules are
    benched (real compile worker: manifest filter + legality + plan on disk),
    the store is published, a winner is picked and exported."""
    from axon import bench_runner
    from axon.bench_runner import BenchStats
    from concurrent.futures import ThreadPoolExecutor
    import numpy as np

    monkeypatch.chdir(tmp_path)
    monkeypatch.setattr(bench_runner, "_make_pipeline_pools",
                        lambda *, n_compile, core_specs: (ThreadPoolExecutor(2), [ThreadPoolExecutor(1)]))
    monkeypatch.setattr(bench_runner, "_visible_gpu_count", lambda: 1)

    def ben(args):
        (x,) = args[4]
        from enzyme_amd.dtypes import to_f32_numpy
        xf = to_f32_numpy(x)
        y = xf / np.sqrt((xf * xf).sum(axis=1, keepdims=True))
        tiles = args[2]
        return BenchStats(1.0 + tiles[0], 1.0 + tiles[0], 1.0, 1.0, 0.0, outputs=(y,))

    monkeypatch.setattr(bench_runner, "_bench_one_artifact", ben)
    with pytest.raises(SystemExit) as e:
        cli.main([str(KERNELS / "rmsnorm"), "--sizes", "32", "1024", "--out", "out/rmsnorm_t32",
                  "--rtol", "1e-2", "--atol", "1e-2"])
    assert e.value.code == 0
    csv_path = tmp_path / "out" / "rmsnorm_t32.csv"
    assert csv_path.is_file()
    assert (tmp_path / "out" / "winners" / "rmsnorm_t32.py").is_file()
    assert (tmp_path / "out" / "winners" / "rmsnorm_t32_case.py").is_file()
    import pandas as pd

    df = pd.read_csv(csv_path)
    timed = df[df["median_ms"].notna()]
    assert len(timed) > 0 and timed["correct"].all()
    # Illegal tuples from the manifest-legal set are "assert" compile rows.
    assert set(df["error"].dropna().unique()) <= {"compile: assert"}
