"""`enzyme_amd.specialize_winner`: the winners/ deliverable step (the
reference's tools/specialize_winner.py rules: bind the tile arguments as
constants, keep the body unchanged, measured only, best wins, --force,
--from-csv), on modules written by this backend's emitter."""

import csv
import importlib.util
import sys

import pytest

from enzyme_amd import hip
from enzyme_amd import specialize_winner as sw
from enzyme_amd.emit import variant_module_text
from tests._specs import load_spec

STEM = "rmsnorm_h1024"
DIMS = {"m": 1024, "n": 1024}


def _setup(tmp_path, medians=((2, 2, 0.0123, "True"), (1, 4, 0.0101, "False"), (4, 1, 0.0150, "True"))):
    spec = load_spec("rmsnorm")
    runs = tmp_path / "out"
    winners = runs / "winners"
    run_dir = runs / STEM
    winners.mkdir(parents=True)
    run_dir.mkdir()
    text = variant_module_text(spec, DIMS, 0, 0, hip.AXON_BF16)
    (run_dir / "rmsnorm__v0_t0.py").write_text(text)
    (winners / f"{STEM}.py").write_text(text)
    case = {"name": STEM, "entry_point": "rmsnorm", "kernel_rel": f"{STEM}.py", "dtype": "bfloat16",
            "shape_args": {"m": 1024, "n": 1024, "TILES_IN_BLOCK_M": 2, "TILES_IN_BLOCK_N": 2},
            "rtol": 0.01, "atol": 0.01}
    (winners / f"{STEM}_case.py").write_text(f'"""case"""\n\nimport numpy\n\nCASE = {case!r}\n')
    with (runs / f"{STEM}.csv").open("w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["hw_variant", "tile_variant", "TILES_M", "TILES_N", "median_ms", "correct"])
        for tm, tn, ms, ok in medians:
            w.writerow([0, 0, tm, tn, ms, ok])
    return runs, winners, tmp_path / "winners"


def test_specialize_binds_tiles_and_keeps_body(tmp_path):
    runs, winners, out = _setup(tmp_path)
    path = sw.specialize_one(STEM, winners, runs, out, tmp_path)
    src = path.read_text()
    assert "def rmsnorm(x):" in src
    assert "    TILES_IN_BLOCK_M = 2\n    TILES_IN_BLOCK_N = 2\n" in src
    assert sw.recorded_us(path) == pytest.approx(12.3)
    assert "measured on" in src and "commit" in src
    # The specialized module runs the library with the bound tiles.
    spec = importlib.util.spec_from_file_location("_spec_winner", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["_spec_winner"] = mod
    spec.loader.exec_module(mod)
    seen = {}
    mod._hip = type("H", (), {"run_variant": staticmethod(lambda meta, ins, tiles: seen.update(t=tiles) or "y")})
    assert mod.rmsnorm("x") == "y" and tuple(seen["t"]) == (2, 2)


def test_best_wins_and_force(tmp_path):
    runs, winners, out = _setup(tmp_path)
    sw.specialize_one(STEM, winners, runs, out, tmp_path)
    with pytest.raises(sw.KeptExisting, match="tie"):
        sw.specialize_one(STEM, winners, runs, out, tmp_path)
    # A slower re-measurement is kept out; --force writes it.
    runs, winners, out = _setup(tmp_path / "b", medians=((2, 2, 0.02, "True"),))
    (out.parent / "winners").mkdir(parents=True, exist_ok=True)
    first = sw.specialize_one(STEM, winners, runs, out, tmp_path)
    first.write_text(first.read_text().replace("20.00 us", "15.00 us"))
    with pytest.raises(sw.KeptExisting, match="slower"):
        sw.specialize_one(STEM, winners, runs, out, tmp_path)
    sw.specialize_one(STEM, winners, runs, out, tmp_path, force=True)
    assert sw.recorded_us(first) == pytest.approx(20.0)


def test_measured_only(tmp_path):
    runs, winners, out = _setup(tmp_path, medians=((2, 2, 0.01, "False"),))
    with pytest.raises(sw.SpecializeError, match="no measurement"):
        sw.specialize_one(STEM, winners, runs, out, tmp_path)
    assert not (out / f"{STEM}.py").exists()


def test_from_csv_picks_fastest_correct_row(tmp_path):
    runs, winners, out = _setup(tmp_path)
    path = sw.specialize_from_csv(STEM, runs, out, tmp_path)
    src = path.read_text()
    # (1, 4) is faster but not correct; (2, 2) is the fastest correct row.
    assert "TILES_IN_BLOCK_M = 2" in src and "TILES_IN_BLOCK_N = 2" in src
    assert sw.recorded_us(path) == pytest.approx(12.3)


def test_rewrite_refuses_unbindable_signatures():
    with pytest.raises(sw.SpecializeError):
        sw.specialize_source("def f(a, b=1):\n    return a\n", "f", {"b": 2})
    with pytest.raises(sw.SpecializeError):
        sw.specialize_source("def f(a):\n    return a\n", "f", {"a": 1})
    with pytest.raises(sw.SpecializeError):
        sw.specialize_source("def f(a):\n    return a\n", "f", {"z": 1})


def test_cli_all(tmp_path, capsys):
    runs, winners, out = _setup(tmp_path)
    assert sw.main(["--all", "--runs-dir", str(runs), "--out-dir", str(out)]) == 0
    assert "WROTE" in capsys.readouterr().out
    assert sw.main(["--all", "--runs-dir", str(runs), "--out-dir", str(out)]) == 0
    assert "KEEP" in capsys.readouterr().out


def test_device_id_from_rocminfo(monkeypatch):
    """An empty Marketing Name line does not swallow the next line."""
    text = ("*******\nAgent 1\n*******\n  Name:                    AMD EPYC\n"
            "*******\nAgent 2\n*******\n  Name:                    gfx950\n"
            "  Marketing Name:          \n  Vendor Name:             AMD\n  Compute Unit:            256\n")

    class R:
        stdout = text

    monkeypatch.setattr(sw.subprocess, "run", lambda *a, **k: R())
    d = sw.device_id()
    assert d.startswith("AMD GPU, gfx950, 256 CUs, 1 GPU agent(s)") and "Vendor" not in d


@pytest.mark.parametrize("path", sorted((sw.REPO / "winners").glob("*.py")), ids=lambda p: p.stem)
def test_committed_winners_are_legal_instantiations(path):
    """Every tracked winner binds a tile tuple the library still accepts for
    its kernel, hw variant and dims, and records a measurement."""
    import ast

    tree = ast.parse(path.read_text())
    meta = next(ast.literal_eval(n.value) for n in tree.body
                if isinstance(n, ast.Assign) and getattr(n.targets[0], "id", "") == "__axon_hip_kernel__")
    fn = next(n for n in tree.body if isinstance(n, ast.FunctionDef))
    tiles = {s.targets[0].id: s.value.value for s in fn.body
             if isinstance(s, ast.Assign) and isinstance(s.value, ast.Constant)}
    values = [tiles[t] for t in meta["tile_args"]]
    dtype = hip.AXON_F32 if meta["kernel"] == "cumsum_probs" else hip.AXON_BF16
    codes = [dtype] * len(meta["input_names"])
    if meta["kernel"] == "rope_llama3":
        codes = [hip.AXON_BF16, hip.AXON_BF16, hip.AXON_F32, hip.AXON_F32]
    st, why = hip.check(meta["kernel"], meta["hw_variant"], values, meta["dims"], codes)
    assert st == hip.AXON_OK, why
    assert sw.recorded_us(path) is not None
