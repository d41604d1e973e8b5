"""`enzyme_amd.verify_specialized` (the reference's tools/verify_specialized.py
contract): the specialized winner must resolve to the same launch as the
parameterized one called with the case's tiles, be legal, and on a GPU give
the same outputs bit for bit, both within the case tolerance of torch_ref."""

import pytest
import torch

from enzyme_amd import hip
from enzyme_amd import specialize_winner as sw
from enzyme_amd import verify_specialized as vs
from enzyme_amd.emit import variant_module_text
from tests._specs import load_spec

STEM = "rmsnorm_h1024"
DIMS = {"m": 1024, "n": 1024}
TILES = {"TILES_IN_BLOCK_M": 2, "TILES_IN_BLOCK_N": 2}


def _setup(tmp_path, spec_tiles=None, hw_variant=0):
    """out/winners/<stem>.py (parameterized) + <stem>_case.py, and the
    specialized module in winners/ (optionally bound to other tiles)."""
    spec = load_spec("rmsnorm")
    runs = tmp_path / "out"
    (runs / "winners").mkdir(parents=True)
    text = variant_module_text(spec, DIMS, hw_variant, 0, hip.AXON_BF16)
    (runs / "winners" / f"{STEM}.py").write_text(text)
    case = {"name": STEM, "entry_point": "rmsnorm", "kernel_rel": f"{STEM}.py", "dtype": "bfloat16",
            "shape_args": {**DIMS, **TILES}, "rtol": 0.01, "atol": 0.01}
    (runs / "winners" / f"{STEM}_case.py").write_text(f'"""case"""\n\nCASE = {case!r}\n')
    out = tmp_path / "winners"
    out.mkdir()
    specialized, _ = sw.specialize_source(text, "rmsnorm", spec_tiles or TILES)
    (out / f"{STEM}.py").write_text(specialized)
    return runs, out


def test_same_plan_and_legal(tmp_path):
    runs, out = _setup(tmp_path)
    r = vs.verify(STEM, runs, out, device=False)
    assert r.same_plan and r.legal and r.ok, vs.format_report(r)
    assert r.plan_param["tiles"] == [2, 2] and r.plan_param["dims"] == [1024, 1024]
    assert "identical" in vs.format_report(r)


def test_other_tiles_are_not_equivalent(tmp_path, capsys):
    runs, out = _setup(tmp_path, spec_tiles={"TILES_IN_BLOCK_M": 4, "TILES_IN_BLOCK_N": 2})
    r = vs.verify(STEM, runs, out, device=False)
    assert not r.same_plan and not r.ok
    assert vs.main([STEM, "--runs-dir", str(runs), "--specialized-dir", str(out), "--no-device"]) == 1
    assert "NOT EQUIVALENT" in capsys.readouterr().out


def test_other_hw_variant_is_not_equivalent(tmp_path):
    runs, out = _setup(tmp_path)
    # Re-emit the specialized module from hw variant 1 with the same tiles.
    other = variant_module_text(load_spec("rmsnorm"), DIMS, 0, 0, hip.AXON_BF16).replace(
        "'hw_variant': 0", "'hw_variant': 1")
    (out / f"{STEM}.py").write_text(sw.specialize_source(other, "rmsnorm", TILES)[0])
    r = vs.verify(STEM, runs, out, device=False)
    assert not r.same_plan and r.plan_spec["hw_variant"] == 1


def test_missing_files_exit_2(tmp_path):
    runs, out = _setup(tmp_path)
    assert vs.main(["nosuchcase", "--runs-dir", str(runs), "--specialized-dir", str(out), "--no-device"]) == 2
    (out / f"{STEM}.py").unlink()
    assert vs.main([STEM, "--runs-dir", str(runs), "--specialized-dir", str(out), "--no-device"]) == 2


@pytest.mark.gpu
def test_device_equivalence(tmp_path):
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    runs, out = _setup(tmp_path)
    r = vs.verify(STEM, runs, out, bench=5, device=True)
    assert r.device and r.correct_param and r.correct_spec and r.bit_identical, vs.format_report(r)
    assert r.legal and r.ok
    assert r.median_us_param > 0 and r.median_us_spec > 0
