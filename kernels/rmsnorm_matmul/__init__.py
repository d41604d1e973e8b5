"""Spec `rmsnorm_matmul`: (x / sqrt(sum x^2)) @ w, sum form without eps
(kernels/rmsnorm_matmul/__init__.py:15-26 of the reference). The reference
package has no `torch_ref`; this one adds it with the same math."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_rmsnorm_matmul
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="rmsnorm_matmul",
    axon_kernel=kernel_rmsnorm_matmul,
    dim_vars=("m", "n", "k"),
    input_specs=(("x", ("m", "k")), ("w", ("k", "n"))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K"),
)
