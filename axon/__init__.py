"""Import name of the reference's host package.

Spec packages written for the reference import `axon.AxonArray` and
`axon.kernel_spec.KernelSpec` (kernels/*/kernel.py, kernels/*/__init__.py),
and its tests import `axon.cli`, `axon.paths`, `axon.bench_runner`, ...
A meta-path finder resolves each of those submodule names to the
corresponding `enzyme_amd` module object (the same object, so module state
and identity checks agree), so the imports work unchanged against this
backend. `python -m axon` runs the command-line driver (`__main__.py`).
"""

import importlib
import importlib.abc
import importlib.util
import sys

from enzyme_amd.axon_array import AxonArray

__all__ = ["AxonArray"]

# The reference's host modules on the hot path, each served by enzyme_amd.
_SERVED = frozenset(
    ("bench_runner", "candidate_filter", "case_gen", "cli", "dtypes", "kernel_spec", "paths", "winner")
)


class _EnzymeAlias(importlib.abc.MetaPathFinder, importlib.abc.Loader):
    """Finds `axon.<name>` for the served names and loads it as the already
    imported (or newly imported) `enzyme_amd.<name>` module."""

    def find_spec(self, fullname, path=None, target=None):
        head, _, name = fullname.partition(".")
        if head == __name__ and name in _SERVED:
            return importlib.util.spec_from_loader(fullname, self)
        return None

    def __init__(self):
        self._specs = {}  # enzyme_amd module name -> its own module spec

    def create_module(self, spec):
        module = importlib.import_module("enzyme_amd." + spec.name.partition(".")[2])
        self._specs[module.__name__] = module.__spec__
        return module

    def exec_module(self, module):
        # The enzyme_amd module is already executed; the import machinery has
        # just set its __spec__ to the alias's, so give it back its own.
        module.__spec__ = self._specs[module.__name__]


if not any(isinstance(f, _EnzymeAlias) for f in sys.meta_path):
    sys.meta_path.insert(0, _EnzymeAlias())
