"""The reference's hot loop end to end on the GPU, through the product code:
`axon <spec> --sizes ... --rtol --atol --out out/<spec>_<case>.csv` emits the
variant modules, applies each module's tile manifest and the budgeted
selection, resolves every key with the real compile worker
(`_compile_one_variant`), times it with the real device worker
(`_bench_one_artifact`), checks it against `baseline_op` and `torch_ref`
(`_check`), appends one terminal row per key to `results.csv`, publishes the
case CSV, picks the winner and exports it with its `_case.py` harness; the
test then launches the exported winner through that harness and compares it
with the harness's own `torch_ref`.

Follows src/axon/bench_runner.py:576-825 (`run_nki_bench`) and
src/axon/winner.py:47-102 (`pick_winner`) of the reference. The worker pools
are in-process executors, as in tests/test_bench_pipeline.py, so nothing is
spawned or exec'd from a process that has touched the GPU."""

from __future__ import annotations

import csv
import importlib.util
import sys
from concurrent.futures import ThreadPoolExecutor

import pytest
import torch

from enzyme_amd import bench_runner, cli, hip
from enzyme_amd.winner import pick_winner
from tests._specs import KERNELS, load_spec

pytestmark = pytest.mark.gpu

# spec, sizes, case id, rtol, atol
CASES = [
    ("rmsnorm_weighted", (256, 4096), "llama_256", 1e-2, 1e-2),
    ("cumsum_probs", (8, 128256), "llama3_vocab_8", 1e-5, 1e-9),
]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


@pytest.fixture
def in_process_pools(monkeypatch):
    def pools(*, n_compile, core_specs):
        return ThreadPoolExecutor(n_compile), [ThreadPoolExecutor(1) for _ in core_specs]

    monkeypatch.setattr(bench_runner, "_make_pipeline_pools", pools)
    monkeypatch.setenv("AXON_SETTLE_MS", "5")
    monkeypatch.setenv("AXON_ROTATE_BYTES", str(64 << 20))
    monkeypatch.setenv("AXON_COMPILE_WORKERS", "2")


def _load(path, name):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("name,sizes,case,rtol,atol", CASES, ids=[c[0] for c in CASES])
def test_cli_sweep_check_store_pick_export(name, sizes, case, rtol, atol, tmp_path, monkeypatch,
                                           in_process_pools):
    print(f"product loop {name} {sizes}", flush=True)
    monkeypatch.chdir(tmp_path)
    out = f"out/{name}_{case}.csv"
    argv = [str(KERNELS / name), "--sizes", *map(str, sizes), "--rtol", str(rtol), "--atol", str(atol),
            "--out", out, "--warmup", "2", "--bench", "10", "--candidate-budget", "3"]
    with pytest.raises(SystemExit) as e:
        cli.main(argv)
    assert e.value.code == 0

    spec = load_spec(name)
    published = tmp_path / out
    with open(published, newline="") as f:
        rows = list(csv.DictReader(f))
    assert rows and list(rows[0]) == bench_runner.result_columns(spec)
    variants = {int(r["hw_variant"]) for r in rows}
    assert variants == set(range(hip.variant_count(name))), f"{name}: hw variants {variants} benched"
    for r in rows:
        key = (r["hw_variant"], [r[c] for c in bench_runner.tile_cols(spec.tile_args)])
        assert r["error"] == "", f"{key}: {r['error']}"
        assert r["correct"] == "True", f"{key}: max_abs_err {r['max_abs_err']}"
        assert 0.0 < float(r["min_ms"]) <= float(r["median_ms"]) <= float(r["max_ms"])
        assert [int(r[d]) for d in spec.dim_vars] == list(sizes)

    winner = pick_winner(published, spec, "median", rtol=rtol, atol=atol)
    assert winner is not None
    assert winner.median_ms == pytest.approx(min(float(r["median_ms"]) for r in rows), rel=1e-12)

    entry = f"{name}_{case}"
    winners = tmp_path / "out" / "winners"
    assert (winners / f"{entry}.py").is_file()
    harness = _load(winners / f"{entry}_case.py", f"_product_loop_case_{name}")
    assert harness.CASE["shape_args"] == {
        **dict(zip(spec.dim_vars, sizes)),
        **dict(zip(spec.tile_args, winner.tile_values)),
    }
    got = harness.run_winner("cuda")
    got = got if isinstance(got, tuple) else (got,)
    torch.cuda.synchronize()
    args = harness.make_inputs(**harness.CASE["shape_args"])
    want = harness.torch_ref(*[args[n] for n in harness.CASE["input_names"]])
    assert len(got) == len(want)
    for i, g in enumerate(got):
        torch.testing.assert_close(g.float().cpu(), want[f"output_{i}"].float(), rtol=rtol, atol=atol)
