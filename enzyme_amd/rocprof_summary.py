"""Per-kernel duration summary of a rocprofv3 `--kernel-trace` run.

Reads either the SQLite database rocprofv3 writes by default
(`<dir>/<name>_results.db`, table `kernels`) or a `*_kernel_stats.csv` from
`--stats --output-format csv`, and prints a Markdown table: calls, average,
min and max duration per kernel, sorted by total time.

    python -m enzyme_amd.rocprof_summary prof/bench_results.db
"""

from __future__ import annotations

import csv
import sqlite3
import sys
from pathlib import Path


def rows_from_db(path: Path) -> list[tuple[str, int, float, float, float, float]]:
    db = sqlite3.connect(str(path))
    try:
        cur = db.execute(
            "select name, count(*), sum(end - start), avg(end - start), min(end - start), "
            "max(end - start) from kernels group by name order by sum(end - start) desc"
        )
        return [(r[0], int(r[1]), r[2] / 1e3, r[3] / 1e3, r[4] / 1e3, r[5] / 1e3) for r in cur]
    finally:
        db.close()


def rows_from_csv(path: Path) -> list[tuple[str, int, float, float, float, float]]:
    out = []
    with path.open(newline="") as f:
        for r in csv.DictReader(f):
            out.append((r["Name"], int(r["Calls"]), float(r["TotalDurationNs"]) / 1e3,
                        float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3))
    out.sort(key=lambda r: -r[2])
    return out


def short(name: str, width: int = 90) -> str:
    name = name.replace("axon::(anonymous namespace)::", "")
    return name if len(name) <= width else name[: width - 3] + "..."


def summarize(path: str | Path) -> str:
    p = Path(path)
    rows = rows_from_db(p) if p.suffix == ".db" else rows_from_csv(p)
    lines = ["| kernel | calls | avg us | min us | max us | total us |", "|---|---:|---:|---:|---:|---:|"]
    for name, calls, total, avg, mn, mx in rows:
        lines.append(f"| `{short(name)}` | {calls} | {avg:.2f} | {mn:.2f} | {mx:.2f} | {total:.1f} |")
    return "\n".join(lines)


if __name__ == "__main__":
    print(summarize(sys.argv[1]))
