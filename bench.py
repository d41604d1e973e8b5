"""Benchmark of the HIP kernel set on one MI355X; prints one JSON line.

A "step" is one launch of the kernel under test over one batch of its
synthetic input. The headline workload is RoPE at the Llama-3-8B shape
(q[1,4096,32,128] + k[1,4096,8,128] bf16, fp32 cos/sin[4096,128] from
theta = 500000), whose metric is achieved HBM GB/s. Every other BASELINE
shape (RMSNorm, cumsum over the vocabulary, the 1024x512x16384 matmul and
its RMSNorm-fused form, causal attention) is measured the same way and
reported under "configs", each against its roofline (HBM bytes or MFMA
FLOPs).

Timing: inputs are resident in HBM before the timed region. Launches rotate
over enough copies of the input/output set to exceed 1 GiB, so the 256 MB
Infinity Cache cannot serve a set that was just touched. Before each
workload's timed region the kernel runs untimed back-to-back launches until
both `--warmup` launches and `--settle-ms` (default 50 ms) of device time
are behind it: after an idle second (the CPU baseline legs leave the GPU
idle) the clocks take about 30 ms of back-to-back launches to settle, and a
launch count alone (the 33 us matmul runs its first launches at 240 us and
its next 25 at 42 us) would time the ramp. The settle each workload got is
reported (`settle_ms`, `settle_launches`). Then exactly `--steps` launches,
captured into one HIP graph, are replayed once between two HIP events on the
stream, bracketed by device syncs; the average launch duration is the
elapsed time / steps. The graph keeps the host's per-launch cost (Python,
ctypes, argument checks: several microseconds) out of the measurement of
kernels that themselves take only 6-16 us.

Correctness: after timing, each workload's outputs are filled with NaN, the
kernel is launched once more, and the result is compared with the oracle
restatement of the spec's torch reference (fp32 on the host) at that
workload's tolerance (rtol = atol = 1e-2 for bf16 outputs; rtol 1e-5,
atol 0 for the fp32 scan of probabilities). Every row carries `allclose`
and `max_abs_err`; the process exits 1 after printing the JSON line if any
row misses.

CPU baseline: the oracle restatement of the same math, timed on the host
cores (torch, all affinity cores) on the full shape of each workload.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--settle-ms 50]
       [--headline-only] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
import warnings
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, 2.5 PFLOP/s
ROTATE_BYTES = 1 << 30

METRIC = "achieved HBM GB/s (% peak) per norm/rope/scan; MFMA TFLOP/s for matmul/attn"

# name, sizes, variant, tiles (picked by the tile sweep on MI355X), bound,
# algorithmic work per launch (bytes for "hbm", FLOPs for "mfma"), the
# correctness tolerance of the row, label. The bound is the larger of the two
# lower limits, bytes / 8 TB/s and FLOPs / 2.5 PFLOP/s: qkv_cte's three
# [16384,8192] residual inputs make it HBM-bound (830 MB: 104 us) although it
# is a GEMM (137 GFLOP: 55 us); its row also reports the MFMA rate (`flops`).
# Tolerances: bf16 outputs rtol = atol = 1e-2; the fp32 scan of probabilities
# rtol 1e-5, atol 0; qkv_cte (bf16, outputs ~N(0,1) after a 8192-deep
# product) rtol = atol = 2e-2, tighter than its own case tolerance (5e-2 /
# 1.5e-1 in eval/sizes.json).
CONFIGS = [
    dict(
        spec="rope_llama3", sizes=(1, 4096, 32, 8, 128), variant=1, tiles=(16, 8), bound="hbm",
        work=88_080_384, rtol=1e-2, atol=1e-2,
        label="RoPE Llama-3-8B: q[1,4096,32,128] k[1,4096,8,128] bf16, cos/sin[4096,128] fp32, theta 500000",
    ),
    dict(
        spec="rmsnorm_weighted", sizes=(2048, 4096), variant=0, tiles=(1, 8), bound="hbm",
        work=33_562_624, rtol=1e-2, atol=1e-2,
        label="RMSNorm x[2048,4096] bf16, weight[4096] bf16, eps 1e-6",
    ),
    dict(
        spec="cumsum_probs", sizes=(64, 128256), variant=2, tiles=(4, 8), bound="hbm",
        work=65_667_072, rtol=1e-5, atol=0.0,
        label="cumsum over vocab: probs[64,128256] fp32 (sorted softmax of N(0,3) logits)",
    ),
    dict(
        spec="matmul_std002", sizes=(1024, 512, 16384), variant=1, tiles=(2, 2, 8), bound="mfma",
        work=2 * 1024 * 512 * 16384, rtol=1e-2, atol=1e-2,
        label="matmul m,n,k = 1024,512,16384 bf16 N(0,0.02), fp32 accumulate",
    ),
    dict(
        spec="rmsnorm_matmul_eps", sizes=(1024, 512, 16384), variant=1, tiles=(2, 2, 8), bound="mfma",
        work=2 * 1024 * 512 * 16384, rtol=1e-2, atol=1e-2,
        label="rmsnorm_matmul m,n,k = 1024,512,16384 bf16, eps 1e-6",
    ),
    dict(
        spec="attention_causal", sizes=(1, 32, 4096, 128), variant=2, tiles=(2, 2, 1, 1), bound="mfma",
        work=137_438_953_472, rtol=1e-2, atol=1e-2,
        label="causal attention Q/K/V [1,32,4096,128] bf16, scale 1/sqrt(128)",
    ),
    dict(
        spec="qkv_cte", sizes=(16384, 512, 8192), variant=3, tiles=(2, 2, 16), bound="hbm",
        work=3 * 16384 * 8192 * 2 + 8192 * 512 * 2 + 16384 * 512 * 2, flops=2 * 16384 * 512 * 8192,
        rtol=2e-2, atol=2e-2,
        label="qkv_cte llama70b: x, mlp_prev, attention_prev [16384,8192] bf16 summed, RMSNorm eps 1e-6, "
              "@ w [8192,512] bf16",
    ),
]

SETTLE_MS = 50.0
_graphs_warm = False
MAX_SETTLE_LAUNCHES = 200_000


def load_spec(name: str):
    from enzyme_amd.cli import _load_spec

    return _load_spec(str(REPO / "kernels" / name))


def timed_launches(launch, n_sets: int, steps: int, warmup: int, settle_ms: float, stream):
    """Settle the clocks, then time `steps` back-to-back launches.

    `launch(i)` enqueues one launch on buffer set i on torch's current stream.
    Untimed launches run first on `stream` until at least `warmup` of them and
    `settle_ms` of device time (HIP events on `stream`) are behind; the chunks
    double so the last one covers at least half the settle period. The timed
    launches are captured into one HIP graph (capture only records; nothing
    runs) and the graph is replayed once between two HIP events on `stream`,
    so the host's per-launch cost (Python, ctypes, argument checks) cannot
    leave the GPU idle between launches of a few-microsecond kernel. Each
    captured launch is an ordinary kernel node over its own buffer set; the
    single-pass scan's launch tags are fresh on this first replay. Returns
    (average us per timed launch, settle ms, settle launches)."""
    import torch

    w0 = torch.cuda.Event(enable_timing=True)
    w1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        w0.record(stream)
        done = 0
        for _ in range(max(0, warmup)):
            launch(done % n_sets)
            done += 1
        w1.record(stream)
        torch.cuda.synchronize()
        chunk = max(1, done)
        while w0.elapsed_time(w1) < settle_ms and done < MAX_SETTLE_LAUNCHES:
            for _ in range(chunk):
                launch(done % n_sets)
                done += 1
            w1.record(stream)
            torch.cuda.synchronize()
            chunk *= 2
    settled = w0.elapsed_time(w1)
    global _graphs_warm
    if not _graphs_warm:
        # The first graph replayed in a process pays a one-time cost (~1.6 ms
        # measured on the causal attention workload): replay a throwaway
        # graph of a few launches first, so no timed replay carries it.
        warm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(warm):
            for i in range(min(4, steps)):
                launch((done + i) % n_sets)
        warm.replay()
        torch.cuda.synchronize()
        del warm
        _graphs_warm = True
    graph = torch.cuda.CUDAGraph()
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        with torch.cuda.graph(graph):
            for i in range(steps):
                launch((done + i) % n_sets)
    if any("empty" in str(w.message) for w in caught):
        raise RuntimeError("the timed launches were not captured (launched off the capture stream)")
    # The capture left the GPU idle for a moment: a short eager burst
    # (2 ms of launches) brings the clocks back before the replay.
    with torch.cuda.stream(stream):
        w0.record(stream)
        burst = 0
        while True:
            for _ in range(max(1, n_sets)):
                launch(burst % n_sets)
                burst += 1
            w1.record(stream)
            torch.cuda.synchronize()
            if w0.elapsed_time(w1) >= 2.0 or burst >= MAX_SETTLE_LAUNCHES:
                break
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
    del graph
    return start.elapsed_time(end) * 1e3 / steps, settled, done


def measure(cfg: dict, steps: int, warmup: int, settle_ms: float):
    """Times `cfg` (see timed_launches) over buffer sets rotating through
    >= 1 GiB, then launches once more on NaN-filled outputs and returns
    (avg_us, settle_ms, settle_launches, fresh outputs on the host as fp32,
    host inputs)."""
    import torch

    from enzyme_amd import hip
    from enzyme_amd.dtypes import to_torch
    from enzyme_amd.kernel_spec import SEED

    spec = load_spec(cfg["spec"])
    dims = dict(zip(spec.dim_vars, cfg["sizes"], strict=True))
    host = spec.make_inputs(**dims, rng=np.random.default_rng(SEED))
    dev = [to_torch(a).cuda() for a in host]
    dvals = [dims[d] for d in spec.dim_vars]
    first = hip.Launcher(spec.name, cfg["variant"], cfg["tiles"], dvals, dev,
                         input_shapes=spec.input_shapes(dims))
    per_set = sum(t.numel() * t.element_size() for t in dev + first.outputs)
    n_sets = max(1, min(64, math.ceil(ROTATE_BYTES / per_set)))
    sets = [first] + [
        hip.Launcher(spec.name, cfg["variant"], cfg["tiles"], dvals, [t.clone() for t in dev])
        for _ in range(n_sets - 1)
    ]
    stream = torch.cuda.current_stream()
    avg_us, settled, launches = timed_launches(
        lambda i: sets[i].launch(), n_sets, steps, warmup, settle_ms, stream)
    for o in first.outputs:
        o.fill_(float("nan"))
    first.launch(stream)
    torch.cuda.synchronize()
    outs = [o.float().cpu() for o in first.outputs]
    del sets, first, dev
    torch.cuda.empty_cache()
    return avg_us, settled, launches, outs, host


def measure_copy(nbytes: int, steps: int, warmup: int, settle_ms: float):
    """The fastest plain device copy reading and writing `nbytes` each, over
    every launch shape of hip.COPY_SHAPES, rotating over >= 1 GiB of buffer
    pairs: the practical HBM ceiling for a streaming kernel moving 2 * nbytes.
    Returns (best us, best shape, {shape: us})."""
    import torch

    from enzyme_amd import hip

    nbytes = max(16, nbytes // 16 * 16)
    n_sets = max(2, min(64, math.ceil(ROTATE_BYTES / (2 * nbytes))))
    sets = [(torch.empty(nbytes, dtype=torch.uint8, device="cuda"),
             torch.empty(nbytes, dtype=torch.uint8, device="cuda")) for _ in range(n_sets)]
    stream = torch.cuda.current_stream()
    by_shape = {}
    for shape in sorted(hip.COPY_SHAPES):
        us, _, _ = timed_launches(lambda i, sh=shape: hip.copy(*sets[i], shape=sh), n_sets, steps,
                                  warmup, settle_ms, stream)
        by_shape[shape] = round(us, 3)
    del sets
    torch.cuda.empty_cache()
    best = min(by_shape, key=by_shape.get)
    return by_shape[best], best, by_shape


def oracle_outputs(cfg: dict, host):
    """fp32 oracle outputs (tuple) of the spec's torch reference on the host."""
    import torch

    import oracle
    from enzyme_amd.dtypes import to_f32_torch

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    with torch.no_grad():
        ref = oracle.ORACLE[cfg["spec"]](*[to_f32_torch(a) for a in host])
    return ref if isinstance(ref, tuple) else (ref,)


def verdict(cfg: dict, gpu_outs, refs) -> dict:
    """allclose of every GPU output against the oracle at the row's tolerance."""
    import torch

    ok = all(
        bool(torch.isfinite(g).all()) and torch.allclose(g, r, rtol=cfg["rtol"], atol=cfg["atol"])
        for g, r in zip(gpu_outs, refs)
    )
    err = max(float((g - r).abs().max()) for g, r in zip(gpu_outs, refs))
    return {"allclose": ok, "rtol": cfg["rtol"], "atol": cfg["atol"], "max_abs_err": err}


def cpu_baseline(cfg: dict, host, runs: int = 10):
    """The oracle on the host cores: (median seconds, threads)."""
    import torch

    import oracle
    from enzyme_amd.dtypes import to_f32_torch

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    fn = oracle.ORACLE[cfg["spec"]]
    args = [to_f32_torch(a) for a in host]
    with torch.no_grad():
        for _ in range(2):
            fn(*args)
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn(*args)
            times.append(time.perf_counter() - t0)
    return float(np.median(times)), torch.get_num_threads()


def roofline(cfg: dict, avg_us: float) -> dict:
    if cfg["bound"] == "hbm":
        achieved = cfg["work"] / (avg_us * 1e-6) / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    else:
        achieved = cfg["work"] / (avg_us * 1e-6) / 1e12
        peak, unit = MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
    return {"bound": cfg["bound"], "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4)}


def traffic_for(kernel: str):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE/WRITE_SIZE and
    scaled against a copy kernel (profiles/traffic_<spec>.json), or None."""
    p = REPO / "profiles" / f"traffic_{kernel}.json"
    if not p.is_file():
        return None
    try:
        return json.loads(p.read_text()).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="minimum device time of untimed launches before each timed region")
    ap.add_argument("--headline-only", action="store_true")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline timing")
    ap.add_argument("--config", action="append", default=[], metavar="SPEC",
                    help="measure only these workload rows (spec names); the headline row is the first")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU; --gpus {args.gpus} is not supported: every kernel here runs "
            "on one MI355X, and no multi-GPU figure is produced",
            file=sys.stderr,
        )
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a visible GPU", file=sys.stderr)
        return 2

    configs = CONFIGS[:1] if args.headline_only else CONFIGS
    if args.config:
        configs = [c for c in CONFIGS if c["spec"] in args.config]
        if not configs:
            print(f"bench.py: no workload named {args.config}", file=sys.stderr)
            return 2
    rows = []
    for cfg in configs:
        us, settled, launches, outs, host = measure(cfg, args.steps, args.warmup, args.settle_ms)
        row = {"spec": cfg["spec"], "label": cfg["label"], "sizes": list(cfg["sizes"]),
               "tiles": list(cfg["tiles"]), "hw_variant": cfg["variant"], "us_per_launch": round(us, 3),
               "settle_ms": round(settled, 2), "settle_launches": launches,
               **roofline(cfg, us), "traffic": traffic_for(cfg["spec"])}
        if "flops" in cfg:
            tf = cfg["flops"] / (us * 1e-6) / 1e12
            row["mfma"] = {"achieved": round(tf, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
        if cfg["bound"] == "hbm":
            cu, shape, by_shape = measure_copy(cfg["work"] // 2, args.steps, args.warmup, args.settle_ms)
            row["copy_us"] = round(cu, 3)
            row["copy_shape"] = shape
            row["copy_us_by_shape"] = by_shape
            row["vs_copy"] = round(cu / us, 4)
        row.update(verdict(cfg, outs, oracle_outputs(cfg, host)))
        if not args.no_cpu:
            runs = 3 if cfg["spec"] in ("attention_causal", "qkv_cte") else 10
            sec, threads = cpu_baseline(cfg, host, runs=runs)
            row["cpu_ms"] = round(sec * 1e3, 3)
            row["cpu_cores"] = threads
        rows.append(row)
        print(f"# {cfg['spec']}: {us:.2f} us, {row['achieved']} {row['unit']} "
              f"({100 * row['frac']:.1f}% of peak), allclose {row['allclose']} "
              f"(max abs err {row['max_abs_err']:.3g}), settle {settled:.1f} ms / {launches} launches",
              file=sys.stderr, flush=True)

    head, hrow = configs[0], rows[0]
    line = {
        "metric": METRIC,
        "value": hrow["achieved"],
        "unit": hrow["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(hrow["us_per_launch"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded make_inputs of the spec package, inputs resident in HBM)",
        "config": {
            "workload": head["label"],
            "spec": head["spec"],
            "sizes": list(head["sizes"]),
            "hw_variant": head["variant"],
            "tiles": list(head["tiles"]),
        },
        "settle_ms": hrow["settle_ms"],
        "settle_launches": hrow["settle_launches"],
        "allclose": hrow["allclose"],
        "roofline": {k: hrow[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")},
    }
    if "copy_us" in hrow:
        line["copy_ceiling"] = {
            "us": hrow["copy_us"],
            "achieved": round(head["work"] / (hrow["copy_us"] * 1e-6) / 1e9, 2),
            "unit": "GB/s",
            "shape": hrow["copy_shape"],
            "what": "fastest of four plain 16-byte-vector copy launch shapes reading and writing half "
                    "the headline's algorithmic bytes each, same buffer rotation: the HBM rate a "
                    "streaming kernel of this size reaches here",
        }
    if "cpu_ms" in hrow:
        line["cpu_baseline"] = {
            "value": round(head["work"] / (hrow["cpu_ms"] * 1e-3) / 1e9, 3),
            "unit": "GB/s",
            "cores": hrow["cpu_cores"],
            "kind": "port",
            "sample": "oracle (fp32 torch restatement of the spec's torch_ref) on the full headline "
                      f"shape, median of 10 runs after 2 warmups: {hrow['cpu_ms']:.2f} ms per pass",
        }
    if not args.headline_only:
        line["configs"] = rows
    print(json.dumps(line))
    failed = [r["spec"] for r in rows if not r["allclose"]]
    if failed:
        print(f"bench.py: outputs outside tolerance for {', '.join(failed)}", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
