"""HBM traffic per launch from rocprofv3 counters, calibrated on a copy.

Two subcommands:

  run SPEC [--steps N]
      Launches one bench.py configuration N times (rotating buffer sets
      exactly as bench.py does) and then `axon_copy` N times over a buffer of
      known size. Meant to run under `rocprofv3 --pmc FETCH_SIZE` and, in a
      second pass, `rocprofv3 --pmc WRITE_SIZE` (one counter group per pass:
      the TCC block holds 4 counters, FETCH_SIZE takes 3 and WRITE_SIZE 2).

  summarize SPEC --fetch CSV --write CSV [--out DIR]
      Reads the two counter-collection CSVs, averages FETCH_SIZE and
      WRITE_SIZE (KiB per dispatch) over the dispatches of the spec's kernel
      and of the copy kernel, scales each by what the copy's known byte count
      says one counted KiB is, and writes `traffic_<spec>.json` (read by
      bench.py as `roofline.traffic`) and `traffic_<spec>.md` into DIR.

Example (on the GPU host, from the repository root):

    cd /tmp && export TMPDIR=/tmp
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d $R/prof/pmc_fetch -o fetch \\
        -- python3 $R/enzyme_amd/traffic.py run rope_llama3
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d $R/prof/pmc_write -o write \\
        -- python3 $R/enzyme_amd/traffic.py run rope_llama3
    python3 $R/enzyme_amd/traffic.py summarize rope_llama3 \\
        --fetch $R/prof/pmc_fetch --write $R/prof/pmc_write --out $R/profiles
"""

from __future__ import annotations

import argparse
import csv
import json
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

COPY_KERNEL = "copy_kernel"

# Kernel-name fragments of each bench configuration's launches.
KERNEL_OF = {
    "rope_llama3": "rope_tok",
    "rmsnorm_weighted": "rowwise_kernel",
    "cumsum_probs": "scan_",
    "matmul_std002": "gemm_kernel",
    "rmsnorm_matmul_eps": "gemm_kernel",
    "attention_causal": "attn_",
    "qkv_cte": "qkv_wide_kernel",
}


def _config(spec: str) -> dict:
    import bench

    for cfg in bench.CONFIGS:
        if cfg["spec"] == spec:
            return cfg
    raise SystemExit(f"no bench configuration named {spec}")


def copy_bytes(cfg: dict) -> int:
    """Bytes the calibration copy reads (and writes): half the configuration's
    algorithmic traffic for HBM-bound kernels, 64 MiB otherwise."""
    if cfg["bound"] == "hbm":
        return (cfg["work"] // 2) // 16 * 16
    return 64 << 20


def run(spec: str, steps: int, variant: int | None = None, tiles: list[int] | None = None) -> None:
    import torch

    import bench
    from enzyme_amd import hip

    cfg = dict(_config(spec))
    if variant is not None:
        cfg["variant"] = variant
    if tiles:
        cfg["tiles"] = tuple(tiles)
    us, _, _, _, _ = bench.measure(cfg, steps, 2, 0.0)
    nbytes = copy_bytes(cfg)
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    for _ in range(steps):
        hip.copy(src, dst)
    torch.cuda.synchronize()
    print(json.dumps({"spec": spec, "hw_variant": cfg["variant"], "tiles": list(cfg["tiles"]), "steps": steps,
                      "us_per_launch": round(us, 3), "copy_bytes": nbytes}), flush=True)


def _counter_rows(path: Path) -> list[dict]:
    files = [path] if path.is_file() else sorted(path.rglob("*counter_collection*.csv"))
    if not files:
        raise SystemExit(f"no counter-collection CSV under {path}")
    rows = []
    for f in files:
        with f.open(newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _col(row: dict, *names: str) -> str:
    lower = {k.lower(): k for k in row}
    for n in names:
        if n.lower() in lower:
            return row[lower[n.lower()]]
    raise KeyError(f"none of {names} in CSV columns {list(row)}")


def per_dispatch(rows: list[dict], counter: str, fragment: str) -> list[float]:
    """Counter value (summed over its instances) per dispatch of kernels whose
    name contains `fragment`."""
    acc: dict[str, float] = {}
    for r in rows:
        if _col(r, "Counter_Name", "counter_name") != counter:
            continue
        if fragment not in _col(r, "Kernel_Name", "kernel_name"):
            continue
        d = _col(r, "Dispatch_Id", "dispatch_id", "Correlation_Id")
        acc[d] = acc.get(d, 0.0) + float(_col(r, "Counter_Value", "counter_value"))
    return list(acc.values())


def summarize(spec: str, fetch: Path, write: Path, out: Path) -> dict:
    cfg = _config(spec)
    frag = KERNEL_OF[spec]
    nbytes = copy_bytes(cfg)
    f_rows, w_rows = _counter_rows(fetch), _counter_rows(write)

    def mean(v):
        if not v:
            raise SystemExit("no matching dispatches in the counter CSV")
        return sum(v) / len(v)

    k_fetch = mean(per_dispatch(f_rows, "FETCH_SIZE", frag))
    k_write = mean(per_dispatch(w_rows, "WRITE_SIZE", frag))
    c_fetch = mean(per_dispatch(f_rows, "FETCH_SIZE", COPY_KERNEL))
    c_write = mean(per_dispatch(w_rows, "WRITE_SIZE", COPY_KERNEL))
    # Bytes per counted KiB, from the copy of known size.
    f_scale = nbytes / c_fetch
    w_scale = nbytes / c_write
    fetched = k_fetch * f_scale
    written = k_write * w_scale
    rec = {
        "spec": spec,
        "kernel_fragment": frag,
        "hbm_bytes_per_launch": int(round(fetched + written)),
        "fetch_bytes_per_launch": int(round(fetched)),
        "write_bytes_per_launch": int(round(written)),
        "algorithmic_bytes": cfg["work"] if cfg["bound"] == "hbm" else None,
        "fetch_kib_per_dispatch": round(k_fetch, 1),
        "write_kib_per_dispatch": round(k_write, 1),
        "copy_bytes": nbytes,
        "copy_fetch_kib": round(c_fetch, 1),
        "copy_write_kib": round(c_write, 1),
        "fetch_bytes_per_counted_kib": round(f_scale, 2),
        "write_bytes_per_counted_kib": round(w_scale, 2),
    }
    out.mkdir(parents=True, exist_ok=True)
    (out / f"traffic_{spec}.json").write_text(json.dumps(rec, indent=1) + "\n")
    return rec


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("spec")
    r.add_argument("--steps", type=int, default=20)
    r.add_argument("--variant", type=int, default=None, help="hw variant (default: bench.py's)")
    r.add_argument("--tiles", type=int, nargs="+", default=None, help="tile tuple (default: bench.py's)")
    s = sub.add_parser("summarize")
    s.add_argument("spec")
    s.add_argument("--fetch", type=Path, required=True)
    s.add_argument("--write", type=Path, required=True)
    s.add_argument("--out", type=Path, default=REPO / "profiles")
    a = ap.parse_args(argv)
    if a.cmd == "run":
        run(a.spec, a.steps, a.variant, a.tiles)
    else:
        print(json.dumps(summarize(a.spec, a.fetch, a.write, a.out), indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
