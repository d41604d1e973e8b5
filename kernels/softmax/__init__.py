"""Spec `softmax`: exp(x) / sum(exp(x)) per row, with no max subtraction
(the reference's definition, kernels/softmax/kernel.py:13-16). The reference
package has no `torch_ref`; this one adds it with the same math."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_softmax
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="softmax",
    axon_kernel=kernel_softmax,
    dim_vars=("m", "n"),
    input_specs=(("x", ("m", "n")),),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"),
)
