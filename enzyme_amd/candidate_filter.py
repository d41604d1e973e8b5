"""Pre-compile filtering of tile candidates from a variant's literal manifest.

The manifest format (`__axon_tile_constraints__ = {"version": 1,
"constraints": ({tile_arg, extent, tile_size, require_divisible}, ...)}`), the
legality rule and the budgeted quality/diversity selection follow
src/axon/candidate_filter.py:13-173. They must agree step for step with the
reference: the selection decides which tile tuples are benched, and a
different pick would make CSVs from the two backends incomparable.
"""

from __future__ import annotations

import ast
import hashlib
import math
from collections.abc import Sequence
from dataclasses import dataclass
from pathlib import Path
from typing import Any

MANIFEST_NAME = "__axon_tile_constraints__"
MANIFEST_VERSION = 1


@dataclass(frozen=True, slots=True)
class TileConstraint:
    """`value * tile_size` must be positive, at most `extent`, and (when
    `require_divisible`) divide `extent`."""

    tile_arg: str
    extent: int
    tile_size: int
    require_divisible: bool

    def rejection_reason(self, value: int) -> str | None:
        block = self.tile_size * value
        if value <= 0:
            return f"{self.tile_arg}={value} is not positive"
        if block > self.extent:
            return f"{self.tile_arg}={value} gives block {block} > extent {self.extent}"
        if self.require_divisible and self.extent % block:
            return (
                f"{self.tile_arg}={value} gives block {block}, which does not "
                f"divide extent {self.extent}"
            )
        return None

    def as_record(self) -> dict[str, Any]:
        return {
            "tile_arg": self.tile_arg,
            "extent": self.extent,
            "tile_size": self.tile_size,
            "require_divisible": self.require_divisible,
        }


def manifest_literal(constraints: Sequence[TileConstraint]) -> str:
    """The Python literal written into a variant module (sorted by tile_arg)."""
    ordered = sorted(constraints, key=lambda c: c.tile_arg)
    return repr(
        {"version": MANIFEST_VERSION, "constraints": tuple(c.as_record() for c in ordered)}
    )


def _manifest_value(tree: ast.Module) -> Any | None:
    for stmt in tree.body:
        if isinstance(stmt, ast.Assign) and any(
            isinstance(t, ast.Name) and t.id == MANIFEST_NAME for t in stmt.targets
        ):
            return ast.literal_eval(stmt.value)
    return None


def read_manifest(module_path: str | Path) -> tuple[TileConstraint, ...]:
    """Parse (never import) a module and return its constraints. Anything
    missing, non-literal, of another version or duplicated fails open: ()."""
    path = Path(module_path)
    if not path.is_file():
        return ()
    try:
        value = _manifest_value(ast.parse(path.read_text(), filename=str(path)))
        if value is None:
            return ()
        if isinstance(value, dict):
            if value.get("version") != MANIFEST_VERSION:
                return ()
            records = value.get("constraints")
        else:  # unversioned tuple of records (early artefacts)
            records = value
        constraints = tuple(TileConstraint(**rec) for rec in records)
    except (OSError, SyntaxError, ValueError, TypeError):
        return ()
    if len({c.tile_arg for c in constraints}) != len(constraints):
        return ()
    return constraints


def rejection_reason(
    tile_args: Sequence[str],
    tile_values: Sequence[int],
    constraints: Sequence[TileConstraint],
) -> str | None:
    """First violated constraint for one tile tuple, matched by argument name."""
    by_name = dict(zip(tile_args, tile_values, strict=True))
    for c in constraints:
        if c.tile_arg not in by_name:
            continue
        reason = c.rejection_reason(int(by_name[c.tile_arg]))
        if reason is not None:
            return reason
    return None


def select_diverse(
    tile_values: Sequence[tuple[int, ...]],
    *,
    budget: int,
    seed: int,
) -> list[tuple[int, ...]]:
    """Deterministically keep at most `budget` legal tuples.

    Each tuple maps to a point in [0,1]^d (log2 of each value over log2 of that
    coordinate's maximum). Anchors (the lexicographic min/max and the
    per-coordinate corner swaps) are seeded first by quality (mean
    coordinate); the rest is filled greedily by 0.65*quality + 0.35*distance
    to the nearest chosen point. Ties break on a sha256 of `seed` and the
    tuple.
    """
    pool = sorted(set(tile_values))
    if budget <= 0 or len(pool) <= budget:
        return pool
    width = len(pool[0])
    hi = tuple(max(t[i] for t in pool) for i in range(width))
    lo = tuple(min(t[i] for t in pool) for i in range(width))

    point = {
        t: tuple(
            math.log2(v) / math.log2(m) if m > 1 else 0.0
            for v, m in zip(t, hi, strict=True)
        )
        for t in pool
    }

    def quality(t: tuple[int, ...]) -> float:
        p = point[t]
        return sum(p) / len(p) if p else 0.0

    def tie(t: tuple[int, ...]) -> int:
        digest = hashlib.sha256(f"{seed}:{','.join(map(str, t))}".encode()).digest()
        return int.from_bytes(digest[:8], "big")

    def dist(a: tuple[int, ...], b: tuple[int, ...]) -> float:
        return math.sqrt(sum((x - y) ** 2 for x, y in zip(point[a], point[b], strict=True)))

    anchors = {pool[0], pool[-1]}
    for i in range(width):
        up = list(lo)
        up[i] = hi[i]
        down = list(hi)
        down[i] = lo[i]
        for cand in (tuple(up), tuple(down)):
            if cand in point:
                anchors.add(cand)
    chosen = sorted(anchors, key=lambda t: (-quality(t), tie(t)))[:budget]

    rest = [t for t in pool if t not in chosen]
    while rest and len(chosen) < budget:
        best = max(
            rest,
            key=lambda t: (
                0.65 * quality(t) + 0.35 * min(dist(t, c) for c in chosen),
                -tie(t),
            ),
        )
        chosen.append(best)
        rest.remove(best)
    return sorted(chosen)
