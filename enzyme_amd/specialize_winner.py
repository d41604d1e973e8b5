"""Bind an exported winner's tile configuration into a standalone module.

Behaviour of the reference's tools/specialize_winner.py (module docstring
1-50, `specialize_source` 96-152, `verify` 155-189, `measured_median_us`
304-340, `decide_write` 351-372, `specialize_from_csv` 375-445,
`specialize_one` 448-510), on this backend's artefacts:

* The exported winner `<runs>/winners/<stem>.py` keeps its `TILES_IN_BLOCK_*`
  parameters; the winning values sit in `<stem>_case.py` under
  `CASE["shape_args"]`. This tool removes every signature parameter the case
  names, binds it as a literal at the top of the body, and checks that the
  rest of the body is unchanged statement for statement (AST dump).
* The result lands in the tracked `winners/<stem>.py` with a provenance
  docstring: shape, tile configuration, measured median, source time, commit
  and the device it was measured on (from `rocminfo`: marketing name, gfx
  target, compute units; `HIP_VISIBLE_DEVICES` when set).
* Measured only: a case without a correct benched row in `<runs>/<stem>.csv`
  is refused. Best wins: an existing artefact is replaced only by a strictly
  faster measurement (at the two decimals the header records); `--force`
  overrides.
* `--from-csv` re-derives the winner from the run CSV (fastest correct row)
  and the emitted candidate module `<runs>/<stem>/<fn>__v<i>_t<j>.py`,
  without the case harness.

Run: `python -m enzyme_amd.specialize_winner <stem> [--runs-dir out]`, or
`--all`. Standard library only; the case module is read with
`ast.literal_eval`, never imported.
"""

from __future__ import annotations

import argparse
import ast
import csv
import getpass
import os
import re
import socket
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
TILE_PREFIX = "TILES_IN_BLOCK_"
HEADER_MEASURED = re.compile(r"^\s*measured\s*:\s*([0-9]+(?:\.[0-9]+)?)\s*us\b", re.MULTILINE)


class SpecializeError(RuntimeError):
    """The winner cannot be specialized; the message says why."""


class KeptExisting(RuntimeError):
    """A stored artefact is at least as fast; nothing was written."""


# ---- source rewrite ---------------------------------------------------------
def read_case(path: Path) -> dict:
    """The literal `CASE = {...}` of a generated case module."""
    tree = ast.parse(path.read_text(), filename=str(path))
    for node in tree.body:
        if isinstance(node, ast.Assign) and any(isinstance(t, ast.Name) and t.id == "CASE" for t in node.targets):
            try:
                return ast.literal_eval(node.value)
            except ValueError as exc:
                raise SpecializeError(f"{path}: CASE is not a literal ({exc})") from exc
    raise SpecializeError(f"{path}: no CASE assignment")


def _entry(tree: ast.Module, name: str) -> ast.FunctionDef:
    found = [n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name == name]
    if not found:
        raise SpecializeError(f"no module-level `def {name}`")
    return found[0]


def specialize_source(src: str, entry: str, values: dict[str, int]) -> tuple[str, list[str]]:
    """`src` with the parameters of `entry` that `values` names removed from
    the signature and bound as constants; returns (source, bound names)."""
    fn = _entry(ast.parse(src), entry)
    a = fn.args
    if a.posonlyargs or a.kwonlyargs or a.vararg or a.kwarg or a.defaults:
        raise SpecializeError(f"{entry}: only plain positional parameters without defaults are supported")
    if any(p.annotation is not None for p in a.args):
        raise SpecializeError(f"{entry}: annotated parameters are not supported")
    params = [p.arg for p in a.args]
    bound = [p for p in params if p in values]
    kept = [p for p in params if p not in values]
    if not bound:
        raise SpecializeError(f"{entry}: no parameter is a case argument; nothing to bind")
    if not kept:
        raise SpecializeError(f"{entry}: every parameter is a case argument")
    first = fn.body[0]
    if first.lineno <= fn.lineno:
        raise SpecializeError(f"{entry}: the body starts on the signature line")
    lines = src.splitlines(keepends=True)
    pad = " " * first.col_offset
    signature = f"{' ' * fn.col_offset}def {entry}({', '.join(kept)}):\n"
    consts = [f"{pad}# Specialized to the benched winner's tile configuration.\n"]
    consts += [f"{pad}{p} = {values[p]!r}\n" for p in bound]
    consts.append("\n")
    out = "".join(lines[: fn.lineno - 1] + [signature] + consts + lines[first.lineno - 1:])
    _check_rewrite(out, entry, kept, bound, fn)
    return out, bound


def _check_rewrite(src: str, entry: str, kept: list[str], bound: list[str], before: ast.FunctionDef) -> None:
    fn = _entry(ast.parse(src), entry)
    if [p.arg for p in fn.args.args] != kept:
        raise SpecializeError(f"{entry}: rewritten signature is not {kept}")
    head, rest = fn.body[: len(bound)], fn.body[len(bound):]
    for stmt, name in zip(head, bound):
        if not (isinstance(stmt, ast.Assign) and len(stmt.targets) == 1
                and isinstance(stmt.targets[0], ast.Name) and stmt.targets[0].id == name
                and isinstance(stmt.value, ast.Constant)):
            raise SpecializeError(f"{entry}: no constant binding for {name}")
    if [ast.dump(s) for s in rest] != [ast.dump(s) for s in before.body]:
        raise SpecializeError(f"{entry}: the rewrite changed the body")


# ---- provenance -------------------------------------------------------------
def device_id() -> str:
    """The GPU the numbers came from, read from `rocminfo` (the first gfx
    agent): marketing name, gfx target and compute-unit count."""
    host = f"{getpass.getuser()}@{socket.gethostname()}"
    visible = os.environ.get("HIP_VISIBLE_DEVICES")
    where = f"host {host}" + (f", HIP_VISIBLE_DEVICES={visible}" if visible else "")
    try:
        out = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=60, check=False).stdout
    except (OSError, subprocess.SubprocessError):
        return f"unknown device ({where})"
    agents = out.split("*******")
    for block in agents:
        name = re.search(r"^[ \t]*Name:[ \t]*(gfx\w+)", block, re.MULTILINE)
        if not name:
            continue
        market = re.search(r"^[ \t]*Marketing Name:[ \t]*(\S[^\n]*)$", block, re.MULTILINE)
        cus = re.search(r"^[ \t]*Compute Unit:[ \t]*(\d+)", block, re.MULTILINE)
        gpus = sum(1 for b in agents if re.search(r"^[ \t]*Name:[ \t]*gfx\w+", b, re.MULTILINE))
        parts = [market.group(1).strip() if market else "AMD GPU", name.group(1)]
        if cus:
            parts.append(f"{cus.group(1)} CUs")
        parts.append(f"{gpus} GPU agent(s)")
        return f"{', '.join(parts)} ({where})"
    return f"no GPU agent in rocminfo ({where})"


def source_commit(repo: Path) -> str:
    """Short HEAD of the tree (AXON_COMMIT wins: a GPU host may lack .git)."""
    env = os.environ.get("AXON_COMMIT", "").strip()
    if env:
        return env
    try:
        head = subprocess.run(["git", "rev-parse", "--short", "HEAD"], cwd=repo, capture_output=True,
                              text=True, timeout=10, check=False)
        if head.returncode != 0 or not head.stdout.strip():
            return "unknown"
        dirty = subprocess.run(["git", "status", "--porcelain", "--untracked-files=no"], cwd=repo,
                               capture_output=True, text=True, timeout=10, check=False)
    except (OSError, subprocess.SubprocessError):
        return "unknown"
    return head.stdout.strip() + ("-dirty" if dirty.stdout.strip() else "")


# ---- measurements -----------------------------------------------------------
def _correct_rows(csv_path: Path) -> list[dict]:
    if not csv_path.is_file():
        raise SpecializeError(f"no measurement: {csv_path} is absent")
    with csv_path.open(newline="") as fh:
        return [r for r in csv.DictReader(fh)
                if r.get("correct", "").strip().lower() == "true" and (r.get("median_ms") or "").strip()]


def _column(param: str) -> str:
    """CSV column of a tile parameter (the CSV drops TILES_IN_BLOCK_ to TILES_)."""
    return "TILES_" + param.removeprefix(TILE_PREFIX).removeprefix("TILES_")


def measured_median_us(csv_path: Path, tiles: dict[str, int]) -> float:
    """Fastest correct median (us) among the CSV rows at exactly these tiles."""
    want = {_column(k): str(v) for k, v in tiles.items()}
    hits = [float(r["median_ms"]) for r in _correct_rows(csv_path)
            if all(r.get(c) == v for c, v in want.items())]
    if not hits:
        raise SpecializeError(f"no measurement: {csv_path.name} has no correct benched row at {want}")
    return min(hits) * 1000.0


def recorded_us(path: Path) -> float | None:
    if not path.is_file():
        return None
    m = HEADER_MEASURED.search(path.read_text())
    return float(m.group(1)) if m else None


def skip_reason(path: Path, new_us: float, force: bool) -> str | None:
    """None when `path` should be (re)written; else why it is kept."""
    old = recorded_us(path)
    if force or old is None:
        return None
    new = round(new_us, 2)
    if new < old:
        return None
    how = "tie" if new == old else "slower"
    return f"kept existing {old:.2f} us; this run measured {new:.2f} us ({how}). Pass --force to overwrite."


def _header(stem: str, how: str, rows: list[tuple[str, str]], places: list[tuple[str, str]]) -> str:
    width = max(len(k) for k, _ in rows + places)
    fmt = lambda kv: f"    {kv[0].ljust(width)} : {kv[1]}\n"  # noqa: E731
    return (f'"""Axon winner for case {stem!r}, specialized to its tile configuration.\n\n'
            f"Generated by enzyme_amd.specialize_winner{how}. Do not edit by hand.\n\n"
            "A standalone kernel module: it takes only tensor inputs; the winning tile\n"
            "configuration is bound as constants in the body, so it cannot disagree with\n"
            "the run it came from.\n\n"
            "Provenance\n----------\n" + "".join(fmt(kv) for kv in rows) +
            "\nWhere the run artefacts live on that host\n"
            "-----------------------------------------\n" + "".join(fmt(kv) for kv in places) + '"""\n\n')


def _stamp(path: Path) -> str:
    return time.strftime("%Y-%m-%d %H:%M:%S %Z", time.localtime(path.stat().st_mtime))


# ---- the two entry paths ----------------------------------------------------
def specialize_one(stem: str, source: Path, runs: Path, out_dir: Path, repo: Path, force: bool = False) -> Path:
    case_path = source / f"{stem}_case.py"
    if not case_path.is_file():
        raise SpecializeError(f"{case_path} not found (is {stem} a head-to-head case?)")
    case = read_case(case_path)
    entry, rel = case.get("entry_point"), case.get("kernel_rel")
    shape_args = dict(case.get("shape_args") or {})
    if not entry or not rel:
        raise SpecializeError(f"{case_path}: CASE lacks entry_point / kernel_rel")
    kernel = (source / rel).resolve()
    if not kernel.is_file():
        raise SpecializeError(f"{kernel} not found")
    new_src, bound = specialize_source(kernel.read_text(), entry, shape_args)
    tiles = {p: int(shape_args[p]) for p in bound}
    dims = {k: v for k, v in shape_args.items() if k not in tiles}
    csv_path = runs / f"{stem}.csv"
    us = measured_median_us(csv_path, tiles)
    out = out_dir / f"{stem}.py"
    why = skip_reason(out, us, force)
    if why:
        raise KeptExisting(why)
    head = _header(stem, "", [
        ("entry point", entry),
        ("shape", ", ".join(f"{k}={v}" for k, v in dims.items()) or "n/a"),
        ("tile config", ", ".join(f"{k}={v}" for k, v in tiles.items())),
        ("measured", f"{us:.2f} us median (on-device, correct)"),
        ("exported", f"{_stamp(kernel)} (mtime of the winner module)"),
        ("commit", source_commit(repo)),
        ("measured on", device_id()),
    ], [("winner module", str(kernel)), ("case metadata", str(case_path)), ("run CSV", str(csv_path)),
        ("variant modules", f"{runs / stem}/")])
    out_dir.mkdir(parents=True, exist_ok=True)
    out.write_text(head + new_src)
    return out


def specialize_from_csv(stem: str, runs: Path, out_dir: Path, repo: Path, force: bool = False) -> Path:
    csv_path, run_dir = runs / f"{stem}.csv", runs / stem
    if not run_dir.is_dir():
        raise SpecializeError(f"{run_dir} not found (was the run cleaned?)")
    mods = sorted(run_dir.glob("*__v*_t*.py"))
    if not mods:
        raise SpecializeError(f"no emitted candidates in {run_dir}")
    entry = mods[0].name.split("__v")[0]
    rows = _correct_rows(csv_path)
    if not rows:
        raise SpecializeError(f"{csv_path}: no correct benched row")
    best = min(rows, key=lambda r: float(r["median_ms"]))
    module = run_dir / f"{entry}__v{best['hw_variant']}_t{best['tile_variant']}.py"
    if not module.is_file():
        raise SpecializeError(f"{module} not found (was {run_dir} cleaned?)")
    fn = _entry(ast.parse(module.read_text()), entry)
    cols = {c: int(v) for c, v in best.items() if c.startswith("TILES_") and v not in (None, "")}
    values = {p.arg: cols[_column(p.arg)] for p in fn.args.args if _column(p.arg) in cols}
    if not values:
        raise SpecializeError(f"{module.name}: no parameter maps to a tile column of {sorted(cols)}")
    us = float(best["median_ms"]) * 1000.0
    out = out_dir / f"{stem}.py"
    why = skip_reason(out, us, force)
    if why:
        raise KeptExisting(why)
    new_src, bound = specialize_source(module.read_text(), entry, values)
    head = _header(stem, " --from-csv", [
        ("entry point", entry),
        ("tile config", ", ".join(f"{p}={values[p]}" for p in bound)),
        ("measured", f"{us:.2f} us median (fastest correct row)"),
        ("emitted", f"{_stamp(module)} (mtime of the candidate module)"),
        ("commit", source_commit(repo)),
        ("measured on", device_id()),
    ], [("candidate", str(module)), ("run CSV", str(csv_path)), ("variant modules", f"{run_dir}/")])
    out_dir.mkdir(parents=True, exist_ok=True)
    out.write_text(head + new_src)
    return out


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("stems", nargs="*", help="case stems, e.g. rmsnorm_h1024")
    ap.add_argument("--all", action="store_true", help="every exported winner (or every run CSV with --from-csv)")
    ap.add_argument("--runs-dir", type=Path, default=Path.cwd() / "out",
                    help="where the run CSVs and run directories are (default ./out)")
    ap.add_argument("--source-dir", type=Path, default=None,
                    help="exported winners (default <runs-dir>/winners)")
    ap.add_argument("--out-dir", type=Path, default=REPO / "winners", help="tracked deliverable directory")
    ap.add_argument("--force", action="store_true", help="overwrite even when this run is not faster")
    ap.add_argument("--from-csv", action="store_true", help="re-derive the winner from the run CSV")
    a = ap.parse_args(argv)
    runs = a.runs_dir.resolve()
    source = (a.source_dir or runs / "winners").resolve()
    if not a.from_csv and not source.is_dir():
        print(f"error: {source} is not a directory (run a bench first)", file=sys.stderr)
        return 2
    if a.all:
        stems = (sorted(p.stem for p in runs.glob("*.csv")) if a.from_csv
                 else sorted(p.name[: -len("_case.py")] for p in source.glob("*_case.py")))
    else:
        stems = list(a.stems)
    if not stems:
        print("error: no stems given (or none found with --all)", file=sys.stderr)
        return 2
    failed = 0
    for stem in stems:
        try:
            if a.from_csv:
                path = specialize_from_csv(stem, runs, a.out_dir, REPO, a.force)
            else:
                path = specialize_one(stem, source, runs, a.out_dir, REPO, a.force)
            print(f"WROTE {stem}: {path}")
        except KeptExisting as exc:
            print(f"KEEP  {stem}: {exc}")
        except SpecializeError as exc:
            print(f"FAIL  {stem}: {exc}", file=sys.stderr)
            failed += 1
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
