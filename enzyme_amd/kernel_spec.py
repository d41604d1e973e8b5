"""The kernel-spec record every `kernels/<name>/` package exports as `SPEC`.

Field set, field order and the `dim_vars` validation follow
src/axon/kernel_spec.py:7-43 of the reference so that a spec package written
for it loads here unchanged (`SEED` is the shared input-generation seed,
src/axon/kernel_spec.py:8).
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import Any

SEED = 42


@dataclass(frozen=True, slots=True)
class KernelSpec:
    name: str
    axon_kernel: Callable[..., Any]
    # Canonical dim order: a make_inputs keyword, a --sizes position and a CSV
    # column each.
    dim_vars: tuple[str, ...]
    input_specs: Sequence[tuple[str, tuple[str | int, ...]]]
    make_inputs: Callable[..., tuple[Any, ...]]
    tile_args: Sequence[str]
    baseline_op: Callable[..., Any] | None = None
    torch_ref: Callable[..., Any] | None = None
    baseline_compiler_args: str = "--model-type=transformer"
    tile_options: Sequence[int] = (1, 2, 4, 8, 16, 32)

    def __post_init__(self) -> None:
        if len(set(self.dim_vars)) != len(self.dim_vars):
            raise ValueError(
                f"kernel '{self.name}': dim_vars has duplicate names: {self.dim_vars}"
            )
        labels = {
            dim
            for _, sym_shape in self.input_specs
            for dim in sym_shape
            if isinstance(dim, str)
        }
        if set(self.dim_vars) != labels:
            raise ValueError(
                f"kernel '{self.name}': dim_vars {set(self.dim_vars)} does not "
                f"match input_specs labels {labels}"
            )

    def input_names(self) -> list[str]:
        return [name for name, _ in self.input_specs]

    def input_shapes(self, dim_sizes: dict[str, int]) -> list[tuple[int, ...]]:
        """Concrete shape of every input for one binding of `dim_vars`."""
        return [
            tuple(dim_sizes[d] if isinstance(d, str) else int(d) for d in shape)
            for _, shape in self.input_specs
        ]
