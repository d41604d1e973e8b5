"""pick_winner / export_winner semantics (src/axon/winner.py:47-166 of the
reference), over fabricated CSVs; no device."""

import importlib.util

import pandas as pd
import pytest

from axon.paths import run_paths
from axon.winner import export_winner, pick_winner
from tests._specs import KERNELS, load_spec

COLS = ["m", "n", "lnc", "sharding", "hw_variant", "tile_variant", "TILES_M", "TILES_N",
        "mean_ms", "median_ms", "min_ms", "max_ms", "std_dev_ms", "correct", "max_abs_err", "error", "mode"]


def row(hw, tile, tm, tn, median, correct=True, err=0.0):
    return {"m": 1024, "n": 1024, "lnc": 1, "sharding": "lnc1", "hw_variant": hw, "tile_variant": tile,
            "TILES_M": tm, "TILES_N": tn, "mean_ms": median + 0.1 if median is not None else None,
            "median_ms": median, "min_ms": median - 0.1 if median is not None else None,
            "max_ms": median, "std_dev_ms": 0.0, "correct": correct, "max_abs_err": err,
            "error": None, "mode": None}


def write(path, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    pd.DataFrame(rows, columns=COLS).to_csv(path, index=False)


@pytest.fixture
def spec():
    return load_spec("rmsnorm")


def test_fastest_correct_wins(tmp_path, spec):
    p = tmp_path / "c.csv"
    write(p, [row(0, 0, 2, 2, 5.0), row(0, 1, 4, 8, 3.0)])
    w = pick_winner(p, spec, "median", rtol=1e-2, atol=1e-2)
    assert (w.hw_variant, w.tile_variant, w.tile_values, w.sizes) == (0, 1, (4, 8), (1024, 1024))


def test_missing_or_untimed_returns_none(tmp_path, spec):
    assert pick_winner(tmp_path / "none.csv", spec, "median", rtol=1, atol=1) is None
    p = tmp_path / "c.csv"
    write(p, [row(0, 0, 1, 1, None, correct=None)])
    assert pick_winner(p, spec, "median", rtol=1, atol=1) is None


def test_wrong_loses_to_slower_correct_and_counts_skips(tmp_path, spec, capsys):
    p = tmp_path / "c.csv"
    write(p, [row(0, 1, 4, 8, 3.0, correct=False, err=9.9), row(0, 0, 2, 2, 5.0),
              row(0, 2, 8, 8, 7.0, correct=False, err=9.9)])
    w = pick_winner(p, spec, "median", rtol=1e-2, atol=1e-2)
    assert w.tile_variant == 0
    assert "skipped 1 faster but incorrect" in capsys.readouterr().out


def test_unverified_is_ranked_and_warned(tmp_path, spec, capsys):
    p = tmp_path / "c.csv"
    write(p, [row(0, 1, 4, 8, 3.0, correct=None, err=None), row(0, 0, 2, 2, 5.0)])
    w = pick_winner(p, spec, "median", rtol=1e-2, atol=1e-2)
    assert w.tile_variant == 1
    assert "correctness unverified" in capsys.readouterr().out


def test_all_wrong_raises_naming_fastest(tmp_path, spec):
    p = tmp_path / "c.csv"
    write(p, [row(1, 2, 4, 8, 3.0, correct=False, err=9.9), row(0, 1, 2, 2, 5.0, correct=False)])
    with pytest.raises(AssertionError, match="failed on-device correctness") as e:
        pick_winner(p, spec, "median", rtol=1e-2, atol=1e-2)
    assert "v1_t2" in str(e.value) and "9.9" in str(e.value) and "rtol=0.01" in str(e.value)


def test_pick_by_min(tmp_path, spec):
    p = tmp_path / "c.csv"
    a = row(0, 0, 1, 1, 5.0)
    a["min_ms"] = 1.0
    write(p, [a, row(0, 1, 2, 2, 3.0)])
    assert pick_winner(p, spec, "min", rtol=1, atol=1).tile_variant == 0


def test_export_writes_module_and_harness(tmp_path, monkeypatch, spec):
    monkeypatch.chdir(tmp_path)
    paths = run_paths(spec, "out/rmsnorm_h1k.csv")
    write(paths.csv, [row(0, 0, 2, 4, 3.0)])
    mod = paths.variant_module("rmsnorm", 0, 0)
    mod.parent.mkdir(parents=True, exist_ok=True)
    mod.write_text("def rmsnorm(x, TILES_IN_BLOCK_M, TILES_IN_BLOCK_N):\n    return x\n")
    w = pick_winner(paths.csv, spec, "median", rtol=1e-2, atol=1e-2)
    export_winner(spec, w, case_id="h1k", kernel_path=KERNELS / "rmsnorm", paths=paths,
                  dtype="bfloat16", rtol=1e-2, atol=1e-2)
    kern = tmp_path / "out" / "winners" / "rmsnorm_h1k.py"
    case = tmp_path / "out" / "winners" / "rmsnorm_h1k_case.py"
    assert kern.read_text() == mod.read_text()
    s = importlib.util.spec_from_file_location("_case_h1k", case)
    m = importlib.util.module_from_spec(s)
    s.loader.exec_module(m)
    assert m.CASE["name"] == "rmsnorm_h1k" and m.CASE["entry_point"] == "rmsnorm"
    assert m.CASE["shape_args"] == {"m": 1024, "n": 1024, "TILES_IN_BLOCK_M": 2, "TILES_IN_BLOCK_N": 4}
    assert m.CASE["input_names"] == ["x"]
    ins = m.make_inputs(m=8, n=16, TILES_IN_BLOCK_M=1, TILES_IN_BLOCK_N=1)
    ref = m.torch_ref(ins["x"])
    assert set(ref) == {"output_0"} and ref["output_0"].shape == (8, 16)
    assert set(m.output_tensors(ins)) == {"output_0"}


def test_export_missing_module_raises(tmp_path, monkeypatch, spec):
    monkeypatch.chdir(tmp_path)
    paths = run_paths(spec, "out/rmsnorm_h1k.csv")
    write(paths.csv, [row(0, 3, 2, 4, 3.0)])
    w = pick_winner(paths.csv, spec, "median", rtol=1e-2, atol=1e-2)
    with pytest.raises(FileNotFoundError, match="winning variant module not found"):
        export_winner(spec, w, case_id="h1k", kernel_path=KERNELS / "rmsnorm", paths=paths,
                      dtype="bfloat16", rtol=1e-2, atol=1e-2)
