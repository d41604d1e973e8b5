"""Spec `rope`: pointwise rotation on the d-major split layout
(kernels/rope/__init__.py:15-33 of the reference): four inputs of shape
(half_d, free), two outputs."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_rope
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="rope",
    axon_kernel=kernel_rope,
    dim_vars=("half_d", "free"),
    input_specs=(
        ("x_even", ("half_d", "free")),
        ("x_odd", ("half_d", "free")),
        ("cos", ("half_d", "free")),
        ("sin", ("half_d", "free")),
    ),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"),
)
