"""Winner selection over a published case CSV, and the winner export.

`pick_winner` follows src/axon/winner.py:47-102 of the reference: sort the
timed rows by the chosen statistic; a row whose `correct` is explicitly false
is skipped; NaN (unverified) is ranked like any other row but warned about;
if every timed row is verified wrong, fail loudly naming the fastest one.
`export_winner` (src/axon/winner.py:105-166) copies the winning variant
module next to a per-case harness module.
"""

from __future__ import annotations

import shutil
from dataclasses import dataclass
from pathlib import Path
from typing import Literal

from enzyme_amd.bench_runner import tile_cols
from enzyme_amd.case_gen import generate_case_module
from enzyme_amd.emit import safe_name
from enzyme_amd.kernel_spec import KernelSpec
from enzyme_amd.paths import RunPaths, _fs_safe

PickBy = Literal["median", "mean", "min"]


@dataclass(frozen=True)
class WinnerRow:
    hw_variant: int
    tile_variant: int
    mean_ms: float | None
    median_ms: float | None
    min_ms: float | None
    sizes: tuple[int, ...]
    tile_values: tuple[int, ...]
    lnc: int = 1
    sharding: str = "lnc1"


def _verified_wrong(correct: object) -> bool:
    """Only an explicit false is wrong; NaN/empty means unverified."""
    import pandas as pd

    if pd.isna(correct):
        return False
    if isinstance(correct, str):
        return correct.strip().lower() in ("false", "0")
    return not bool(correct)


def _tag(row) -> str:
    return f"v{int(row['hw_variant'])}_t{int(row['tile_variant'])}"


def pick_winner(
    csv_path: Path, spec: KernelSpec, pick_by: PickBy, *, rtol: float, atol: float
) -> WinnerRow | None:
    """Fastest timed row that is not verified incorrect (None when the CSV
    is missing or has no timed rows)."""
    import pandas as pd

    if not csv_path.is_file():
        return None
    df = pd.read_csv(csv_path)
    col = f"{pick_by}_ms"
    if col not in df.columns:
        return None
    timed = df[df[col].notna()]
    if timed.empty:
        return None
    ranked = timed.sort_values(col, kind="stable")
    wrong = [bool(_verified_wrong(c)) for c in ranked["correct"]]
    if all(wrong):
        worst = ranked.iloc[0]
        raise AssertionError(
            f"{spec.name} winner {_tag(worst)} failed on-device correctness: "
            f"max_abs_err={worst['max_abs_err']} exceeds rtol={rtol} atol={atol}"
        )
    first_ok = wrong.index(False)
    row = ranked.iloc[first_ok]
    tag = _tag(row)
    if first_ok:
        print(f"[info] {spec.name} skipped {first_ok} faster but incorrect variant(s); winner is {tag}")
    if pd.isna(row["correct"]):
        print(
            f"[warn] {spec.name} winner {tag} correctness unverified "
            f"(no baseline_op or no device outputs); shipping unchecked"
        )
    cols = tile_cols(spec.tile_args)
    return WinnerRow(
        hw_variant=int(row["hw_variant"]),
        tile_variant=int(row["tile_variant"]),
        mean_ms=float(row["mean_ms"]),
        median_ms=float(row["median_ms"]),
        min_ms=float(row["min_ms"]),
        sizes=tuple(int(row[c]) for c in spec.dim_vars),
        tile_values=tuple(int(row[c]) for c in cols),
        lnc=int(row["lnc"]) if "lnc" in row else 1,
        sharding=str(row["sharding"]) if "sharding" in row else "lnc1",
    )


def export_winner(
    spec: KernelSpec,
    winner: WinnerRow,
    *,
    case_id: str,
    kernel_path: Path | str,
    paths: RunPaths,
    dtype: str,
    rtol: float,
    atol: float,
) -> None:
    """Copy the winning module to `winners/<name>_<case>.py` and write its
    per-case harness `winners/<name>_<case>_case.py` beside it."""
    entry = f"{spec.name}_{case_id}"
    print(f"\n=== export {entry} ===")
    print(
        f"  winner: hw_variant={winner.hw_variant}, tile_variant={winner.tile_variant}, "
        f"median_ms={winner.median_ms}, mean_ms={winner.mean_ms}, min_ms={winner.min_ms}"
    )
    fn = safe_name(spec.name)
    if winner.lnc >= 2:
        src = paths.spmd_variant_module(
            fn, winner.hw_variant, winner.tile_variant, _fs_safe(winner.sharding)
        )
    else:
        src = paths.variant_module(fn, winner.hw_variant, winner.tile_variant)
    if not src.is_file():
        raise FileNotFoundError(
            f"winning variant module not found at {src}; the CSV row references a "
            f"variant whose source file is missing; re-run axon."
        )
    dst = paths.winner_kernel(entry)
    dst.parent.mkdir(parents=True, exist_ok=True)
    shutil.copyfile(src, dst)
    print(f"  wrote {dst}")
    shape_args = dict(zip(spec.dim_vars, winner.sizes, strict=True))
    tiles = {a: int(v) for a, v in zip(spec.tile_args, winner.tile_values, strict=True)}
    case_path = paths.winner_case(entry)
    generate_case_module(
        spec, kernel_path, dtype, case_path, name=entry, entry_point=fn,
        shape_args={**shape_args, **tiles}, rtol=rtol, atol=atol,
    )
    print(f"  wrote {case_path}")
