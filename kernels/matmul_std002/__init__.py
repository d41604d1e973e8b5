"""Spec `matmul_std002`: the same product as `matmul`, with both operands
drawn from N(0, 0.02^2) (a transformer weight-init scale). Not in the
reference, whose `matmul` scales x by 1/sqrt(k) and keeps w ~ N(0, 1)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_matmul_std002
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="matmul_std002",
    axon_kernel=kernel_matmul_std002,
    dim_vars=("m", "n", "k"),
    input_specs=(("a", ("m", "k")), ("b", ("k", "n"))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K"),
)
