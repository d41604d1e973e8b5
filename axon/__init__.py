"""Import name of the reference's host package.

Spec packages written for the reference import `axon.AxonArray` and
`axon.kernel_spec.KernelSpec` (kernels/*/kernel.py, kernels/*/__init__.py),
and its tests import `axon.cli`, `axon.paths`, `axon.bench_runner`, ...
Each submodule here re-exports the corresponding `enzyme_amd` module so those
imports resolve to this backend unchanged.
"""

from enzyme_amd.axon_array import AxonArray

__all__ = ["AxonArray"]
