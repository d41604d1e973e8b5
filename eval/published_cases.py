"""The reference's published cases on MI355X, beside the reference's numbers.

The reference publishes 13 measurements, the medians of its specialized
Trainium2 winners (winners/<case>.py:12-17 of the reference, e.g.
winners/rmsnorm_h1024.py:14 "34.53 us median"). This script measures the
same cases here in two steps:

  sweep   runs the product CLI on each case (`python -m axon <spec> --sizes
          ... --rtol --atol --candidate-budget 0 --out <dir>/<case>.csv`):
          every legal tile tuple of every hw variant is benched with the
          reference's protocol (20 warmup launches, then 100 timed launches,
          median per-launch time; plus this backend's 50 ms clock settle),
          checked, and the winner picked and exported;
  report  reads each case CSV, takes the winner's CLI median, re-times that
          winner in this process as bench.py does (buffer rotation over 1 GiB,
          clock settle, one HIP-graph replay of 200 launches) and checks it
          against the spec's fp32 torch reference at the case tolerance,
          then prints a Markdown table beside the trn2 medians.

    python eval/published_cases.py sweep --dir gpurun_out/published
    python eval/published_cases.py report --dir gpurun_out/published

`report` runs in one process, so `rocprofv3 --kernel-trace --stats --
python3 eval/published_cases.py report ...` gives the kernel durations of
the same launches.
"""

from __future__ import annotations

import argparse
import json
import math
import subprocess
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

# case, spec, sizes, dtype (None = the spec's default), rtol, atol (the
# reference's eval/sizes.json entry), trn2 median us (winners/<case>.py:14),
# work per launch, unit ("B" = algorithmic HBM bytes, "FLOP").
CASES = [
    ("rmsnorm_h1024", "rmsnorm", (1024, 1024), None, 1e-2, 1e-2, 34.53, 2 * 1024 * 1024 * 2, "B"),
    ("rmsnorm_h4096", "rmsnorm", (1024, 4096), None, 1e-2, 1e-2, 76.18, 2 * 1024 * 4096 * 2, "B"),
    ("rmsnorm_h8192", "rmsnorm", (128, 8192), None, 1e-2, 1e-2, 35.83, 2 * 128 * 8192 * 2, "B"),
    ("layernorm_llama70b", "layernorm", (128, 8192), None, 2e-2, 2e-2, 48.43, 2 * 128 * 8192 * 2, "B"),
    ("rope_llama3_8b", "rope", (128, 4096), None, 7.8125e-3, 2e-2, 31.89, 6 * 128 * 4096 * 2, "B"),
    ("rope_gqa_long", "rope", (128, 32768), None, 7.8125e-3, 2e-2, 140.77, 6 * 128 * 32768 * 2, "B"),
    ("cumsum_fast_small", "cumsum", (1024, 1024), None, 1e-3, 1e-3, 32.20, 2 * 1024 * 1024 * 4, "B"),
    ("cumsum_fast_small_bf16", "cumsum", (1024, 1024), "bfloat16", 1e-2, 1e-2, 24.03,
     2 * 1024 * 1024 * 2, "B"),
    ("cumsum_nucleus", "cumsum", (128, 32768), None, 1e-3, 1e-3, 88.96, 2 * 128 * 32768 * 4, "B"),
    ("cumsum_fast_large", "cumsum", (4096, 4096), None, 1e-3, 1e-3, 343.46, 2 * 4096 * 4096 * 4, "B"),
    ("cumsum_llama3_vocab", "cumsum", (128, 128256), None, 1e-3, 1e-3, 327.00, 2 * 128 * 128256 * 4, "B"),
    ("cumsum_qwen_vocab", "cumsum", (128, 151936), None, 1e-3, 1e-3, 385.84, 2 * 128 * 151936 * 4, "B"),
    ("attention_nkilib_d128", "attention_nkilib", (1024, 128), None, 5e-2, 5e-2, 41.32,
     4 * 1024 * 1024 * 128, "FLOP"),
]


def _case_id(case: str, spec: str) -> str:
    return case[len(spec) + 1:]


def sweep(out_dir: Path, only: list[str]) -> int:
    """One CLI run per case; the CLI is a child process (spawned workers)."""
    out_dir.mkdir(parents=True, exist_ok=True)
    for case, spec, sizes, dtype, rtol, atol, *_ in CASES:
        if only and case not in only:
            continue
        csv = out_dir / f"{spec}_{_case_id(case, spec)}.csv"
        cmd = [sys.executable, "-m", "axon", str(REPO / "kernels" / spec), "--sizes", *map(str, sizes),
               "--rtol", str(rtol), "--atol", str(atol), "--candidate-budget", "0", "--out", str(csv)]
        if dtype:
            cmd += ["--dtype", dtype]
        print(f"== {case}: {' '.join(cmd[2:])}", flush=True)
        log = out_dir / f"{case}.log"
        with open(log, "w") as f:
            rc = subprocess.run(cmd, cwd=str(REPO), stdout=f, stderr=subprocess.STDOUT).returncode
        print(f"   exit {rc} (log {log})", flush=True)
        if rc != 0:
            return rc
    return 0


def _time_winner(spec_name, sizes, dtype, variant, tiles, rtol, atol, steps=200):
    import torch

    import bench
    from enzyme_amd import hip
    from enzyme_amd.dtypes import resolve, to_f32_torch, to_torch
    from enzyme_amd.kernel_spec import SEED

    spec = bench.load_spec(spec_name)
    dims = dict(zip(spec.dim_vars, sizes, strict=True))
    kw = {"dtype": resolve(dtype)} if dtype else {}
    host = spec.make_inputs(**dims, **kw, rng=np.random.default_rng(SEED))
    dev = [to_torch(a).cuda() for a in host]
    dvals = [dims[d] for d in spec.dim_vars]
    first = hip.Launcher(spec.name, variant, tiles, dvals, dev, input_shapes=spec.input_shapes(dims))
    per_set = sum(t.numel() * t.element_size() for t in dev + first.outputs)
    n_sets = max(1, min(64, math.ceil(bench.ROTATE_BYTES / per_set)))
    sets = [first] + [hip.Launcher(spec.name, variant, tiles, dvals, [t.clone() for t in dev])
                      for _ in range(n_sets - 1)]
    stream = torch.cuda.current_stream()
    us, _, _ = bench.timed_launches(lambda i: sets[i].launch(), n_sets, steps, 20, bench.SETTLE_MS, stream)
    for o in first.outputs:
        o.fill_(float("nan"))
    first.launch()
    torch.cuda.synchronize()
    want = spec.torch_ref(*[to_f32_torch(a) for a in host])
    want = want if isinstance(want, tuple) else (want,)
    ok = all(torch.allclose(g.float().cpu(), w.float(), rtol=rtol, atol=atol)
             for g, w in zip(first.outputs, want))
    del sets, first, dev
    torch.cuda.empty_cache()
    return us, ok


def report(out_dir: Path, only: list[str]) -> int:
    from enzyme_amd.winner import pick_winner

    import bench

    rows = []
    print("| case | shape | winner (hw variant, tiles) | CLI median us | graph-replay us | achieved | "
          "MI355X % of peak | trn2 median us | trn2 / MI355X | correct |")
    print("|---|---|---|---:|---:|---:|---:|---:|---:|---|")
    for case, spec_name, sizes, dtype, rtol, atol, trn2_us, work, unit in CASES:
        if only and case not in only:
            continue
        spec = bench.load_spec(spec_name)
        csv = out_dir / f"{spec_name}_{_case_id(case, spec_name)}.csv"
        w = pick_winner(csv, spec, "median", rtol=rtol, atol=atol)
        if w is None:
            print(f"| {case} | no results in {csv} |")
            continue
        us, ok = _time_winner(spec_name, sizes, dtype, w.hw_variant, w.tile_values, rtol, atol)
        if unit == "B":
            rate, peak, runit = work / (us * 1e-6) / 1e9, bench.HBM_PEAK_GBS, "GB/s"
        else:
            rate, peak, runit = work / (us * 1e-6) / 1e12, bench.MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
        cli_us = w.median_ms * 1e3
        rows.append({"case": case, "spec": spec_name, "sizes": list(sizes), "dtype": dtype,
                     "hw_variant": w.hw_variant, "tiles": list(w.tile_values), "cli_median_us": cli_us,
                     "graph_us": us, "achieved": rate, "unit": runit, "frac": rate / peak,
                     "trn2_median_us": trn2_us, "speedup_vs_trn2": trn2_us / us, "correct": ok})
        shape = "x".join(map(str, sizes)) + (f" {dtype}" if dtype else "")
        print(f"| {case} | {shape} | v{w.hw_variant} {tuple(w.tile_values)} | {cli_us:.2f} | {us:.2f} | "
              f"{rate:.1f} {runit} | {100 * rate / peak:.1f}% | {trn2_us:.2f} | {trn2_us / us:.1f}x | {ok} |",
              flush=True)
    (out_dir / "published_report.json").write_text(json.dumps(rows, indent=1))
    return 0 if all(r["correct"] for r in rows) else 1


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("step", choices=("sweep", "report"))
    ap.add_argument("--dir", default="out/published")
    ap.add_argument("--case", action="append", default=[], help="limit to these case names")
    args = ap.parse_args(argv)
    out = Path(args.dir).resolve()
    return sweep(out, args.case) if args.step == "sweep" else report(out, args.case)


if __name__ == "__main__":
    sys.exit(main())
