"""The `make <kernel>_<case>` flow: eval/gen_size_targets.py's fragment and the
Makefile around it (the reference's eval/gen_size_targets.py:25-86 and
Makefile:39-46, 98-113)."""

import json
import shutil
import subprocess
import sys

import pytest

from tests._specs import REPO

sys.path.insert(0, str(REPO / "eval"))
import gen_size_targets as gst  # noqa: E402

CASES = json.loads((REPO / "eval" / "sizes.json").read_text())


def _cases():
    return [(k, c, cfg) for k, per in CASES.items() if not k.startswith("_")
            for c, cfg in per.items() if not c.startswith("_")]


def test_every_case_has_a_target_with_its_whole_command_line():
    frag = gst.fragment(CASES)
    lines = frag.splitlines()
    for kernel, cid, cfg in _cases():
        target = f"{kernel}_{cid}"
        i = lines.index(f"out/{target}.csv: $(wildcard kernels/{kernel}/*.py) eval/sizes.json $(AXON_LIB)")
        cmd = lines[i + 1]
        assert cmd.startswith(f"\t$(PYTHON) -m axon $(AXON_ARGS) kernels/{kernel} --sizes ")
        assert cmd.endswith(" --out $@")
        argv = cmd.split()
        sizes = argv[argv.index("--sizes") + 1:]
        sizes = sizes[: next((j for j, a in enumerate(sizes) if a.startswith("--")), len(sizes))]
        assert [int(s) for s in sizes] == list(cfg["sizes"])
        assert ("--dtype" in argv) == ("dtype" in cfg)
        if "dtype" in cfg:
            assert argv[argv.index("--dtype") + 1] == cfg["dtype"]
        h2h = "rtol" in cfg and "atol" in cfg
        if h2h:
            assert float(argv[argv.index("--rtol") + 1]) == cfg["rtol"]
            assert float(argv[argv.index("--atol") + 1]) == cfg["atol"]
            assert lines[i + 2] == f"\t-$(PYTHON) -m enzyme_amd.specialize_winner {target}"
        else:
            assert "--rtol" not in argv and lines[i + 2] == ""
        assert f"{target}: out/{target}.csv" in lines
    every = next(ln for ln in lines if ln.startswith("CASE_TARGETS := ")).split()[2:]
    assert every == [f"{k}_{c}" for k in sorted(k for k in CASES if not k.startswith("_"))
                     for c in CASES[k] if not c.startswith("_")]


def test_lnc_split_and_no_specialize_for_sharded_cases():
    data = {"_comment": {}, "mm": {"a": {"sizes": [4, 4, 4], "rtol": 0.1, "atol": 0.1},
                                   "b": {"sizes": [8, 8, 8], "lnc": 2, "rtol": 0.1, "atol": 0.1},
                                   "_skip": {"sizes": [1]}}}
    frag = gst.fragment(data)
    assert "LNC1_TARGETS := mm_a\n" in frag and "LNC2_TARGETS := mm_b\n" in frag
    assert "CASES_mm := mm_a mm_b\n" in frag
    assert "--sizes 8 8 8 --rtol 0.1 --atol 0.1 --lnc 2 --out $@" in frag
    assert "specialize_winner mm_b" not in frag and "specialize_winner mm_a" in frag
    assert "_skip" not in frag


@pytest.fixture()
def tree(tmp_path):
    if shutil.which("make") is None:
        pytest.skip("make is not installed")
    for name in ("Makefile",):
        shutil.copy(REPO / name, tmp_path / name)
    shutil.copytree(REPO / "eval", tmp_path / "eval", ignore=shutil.ignore_patterns("__pycache__"))
    for name in ("kernels", "enzyme_amd", "include"):
        (tmp_path / name).symlink_to(REPO / name)
    return tmp_path


def _make(tree, *args):
    # AXON_LIB is pointed at an existing file so the dry run never asks for a rebuild.
    return subprocess.run(["make", "-n", f"AXON_LIB={REPO / 'Makefile'}", *args], cwd=tree,
                          capture_output=True, text=True, timeout=60)


def test_make_dry_run_runs_the_driver_then_the_specialiser(tree):
    r = _make(tree, "rmsnorm_h4096")
    assert r.returncode == 0, r.stderr
    out = r.stdout.splitlines()
    assert "python3 -m axon  kernels/rmsnorm --sizes 1024 4096 --rtol 0.01 --atol 0.01 --out out/rmsnorm_h4096.csv" in out
    assert out[-1] == "python3 -m enzyme_amd.specialize_winner rmsnorm_h4096"
    r = _make(tree, "matmul_sq1k", "AXON_ARGS=--candidate-budget 2")
    assert r.returncode == 0, r.stderr
    assert r.stdout.splitlines()[-1] == ("python3 -m axon --candidate-budget 2 kernels/matmul "
                                         "--sizes 1024 1024 1024 --out out/matmul_sq1k.csv")


def test_bare_kernel_lists_its_cases_and_fails(tree):
    r = subprocess.run(["make", "rmsnorm"], cwd=tree, capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "Pick a case for 'rmsnorm'" in r.stdout
    assert [ln.strip() for ln in r.stdout.splitlines() if ln.startswith("  make ")] == [
        f"make rmsnorm_{c}" for c in CASES["rmsnorm"] if not c.startswith("_")]
