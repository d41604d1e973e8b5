"""Spec `rmsnorm`: sum-form RMS normalisation of each row (no eps, no weight).

Spec surface as in the reference's kernels/rmsnorm/__init__.py:15-24
(dim_vars (m, n), one input x[m, n], tile args M/N)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_rmsnorm
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="rmsnorm",
    axon_kernel=kernel_rmsnorm,
    dim_vars=("m", "n"),
    input_specs=(("x", ("m", "n")),),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"),
)
