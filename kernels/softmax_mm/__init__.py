"""Spec `softmax_mm`: softmax over each row of x (bare exp / sum, no max
subtraction), then @ w (kernels/softmax_mm/__init__.py:14-27 of the
reference). The reference package has no torch_ref; this one adds it with
the same math."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_softmax_matmul
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="softmax_mm",
    axon_kernel=kernel_softmax_matmul,
    dim_vars=("m", "n", "k"),
    input_specs=(("x", ("m", "k")), ("w", ("k", "n"))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K"),
    tile_options=(1, 2, 4, 8, 16),
)
