"""`--mode baseline` (the reference's src/axon/bench_runner.py:828-889
benches the spec's baseline on the device): here the spec's torch_ref runs
eagerly on the GPU through torch-ROCm, or on the host CPU cores when no GPU
is visible; one row per run lands in the baseline CSV with a `device`
column."""

import pandas as pd
import pytest
import torch

from enzyme_amd import bench_runner
from enzyme_amd.paths import run_paths
from tests._specs import load_spec


def _run(tmp_path, name, dims):
    spec = load_spec(name)
    paths = run_paths(spec, str(tmp_path / "out" / f"{name}_t.csv"))
    csv = bench_runner.run_baseline(spec, dims, warmup=1, bench=3, paths=paths)
    return pd.read_csv(csv)


def test_baseline_on_cpu_without_gpu(tmp_path, monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    df = _run(tmp_path, "rmsnorm", {"m": 8, "n": 64})
    assert list(df["device"]) == ["cpu"] and df["cpu_threads"].iloc[0] >= 1
    assert df["median_ms"].iloc[0] > 0 and list(df[["m", "n"]].iloc[0]) == [8, 64]


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "dims"), [("matmul_std002", {"m": 256, "n": 128, "k": 512}),
                                            ("attention_causal", {"b": 1, "h": 2, "s": 256, "d": 128}),
                                            ("rope_llama3", {"b": 1, "s": 64, "hq": 4, "hkv": 2, "d": 128})])
def test_baseline_on_gpu(tmp_path, name, dims):
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    df = _run(tmp_path, name, dims)
    assert df["device"].iloc[0].startswith("gpu:")
    assert df["median_ms"].iloc[0] > 0
