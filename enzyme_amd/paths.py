"""Every per-run path, derived from one CSV path.

Same derivation rules as src/axon/paths.py:19-92 (the run stem `out/<stem>`
names `out/<stem>.csv` and the run dir `out/<stem>/`), so split
`--phase emit` / `--phase bench` runs and existing Makefiles agree on where
things live. The per-key artefact of this backend is a launch plan
(`kernel.plan.json`) rather than a NEFF; its directory naming is unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

ARTIFACT_NAME = "kernel.plan.json"


def out_dir() -> Path:
    """Where generated artefacts go."""
    return Path.cwd() / "out"


def _fs_safe(tag: str) -> str:
    """Filesystem-safe form of a sharding tag (`shard=k:P+` -> `shard_k_Pplus`)."""
    return tag.replace("=", "_").replace(":", "_").replace("+", "plus").replace("#", "")


@dataclass(frozen=True, slots=True)
class RunPaths:
    """Only the absolute CSV path is stored; every other path derives from it."""

    csv: Path

    @property
    def run_dir(self) -> Path:
        return self.csv.with_suffix("")

    @property
    def results(self) -> Path:
        """Durable per-key row store, published to `csv` on full coverage."""
        return self.run_dir / "results.csv"

    @property
    def baseline_dir(self) -> Path:
        return self.run_dir.parent / ("baseline_" + self.run_dir.name)

    @property
    def baseline_csv(self) -> Path:
        return self.baseline_dir.parent / (self.baseline_dir.name + ".csv")

    @property
    def winners_dir(self) -> Path:
        return self.csv.parent / "winners"

    def variant_module(self, fn_name: str, i: int, j: int) -> Path:
        return self.run_dir / f"{fn_name}__v{i}_t{j}.py"

    def spmd_variant_module(self, fn_name: str, i: int, j: int, plan_tag: str) -> Path:
        return self.run_dir / f"{fn_name}__v{i}_t{j}_{plan_tag}.py"

    def artifact_dir(self, i: int, j: int, tile_values, plan_tag: str = "") -> Path:
        tile_tag = "_".join(map(str, tile_values))
        suffix = f"_{_fs_safe(plan_tag)}" if plan_tag else ""
        return self.run_dir / f"__v{i}_t{j}{suffix}_tiles_{tile_tag}"

    def artifact(self, i: int, j: int, tile_values, plan_tag: str = "") -> Path:
        return self.artifact_dir(i, j, tile_values, plan_tag) / ARTIFACT_NAME

    def neff(self, i: int, j: int, tile_values, plan_tag: str = "") -> Path:
        """The reference's name for the per-key artefact path; kept so callers
        written against it still resolve (the file is a launch plan here)."""
        return self.artifact_dir(i, j, tile_values, plan_tag) / "kernel.neff"

    def winner_kernel(self, entry_name: str) -> Path:
        return self.winners_dir / f"{entry_name}.py"

    def winner_case(self, entry_name: str) -> Path:
        return self.winners_dir / f"{entry_name}_case.py"


def run_paths(spec, out: str | None) -> RunPaths:
    """`out` is the run stem; the `.csv` suffix is optional; a trailing slash
    names a container directory for the default `nki_<name>.csv`; omitted,
    the stem is `out/nki_<name>`. The CSV path is made absolute so spawned
    workers (own cwd) derive identical paths."""
    default_name = f"nki_{spec.name}.csv"
    if out is None:
        csv = out_dir() / default_name
    elif out.endswith("/"):
        csv = Path(out) / default_name
    else:
        p = Path(out)
        csv = p if p.suffix == ".csv" else p.with_name(p.name + ".csv")
    return RunPaths(csv=csv.resolve())
