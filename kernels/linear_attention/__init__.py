"""Spec `linear_attention`: out = q (keyᵀ v), the unnormalised core of global
linear attention with an identity feature map (the reference's
kernels/linear_attention/__init__.py:14-37). Input `key` keeps the
reference's name (`k` is a block-loop name in the emitted modules)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_linear_attention
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="linear_attention",
    axon_kernel=kernel_linear_attention,
    dim_vars=("sq", "sk", "dk", "dv"),
    input_specs=(("q", ("sq", "dk")), ("key", ("sk", "dk")), ("v", ("sk", "dv"))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K", "TILES_IN_BLOCK_P"),
    tile_options=(1, 2, 4, 8, 16),
)
