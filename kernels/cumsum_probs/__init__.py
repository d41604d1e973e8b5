"""Spec `cumsum_probs`: the nucleus-sampling scan, an inclusive prefix sum
over each row of sorted (descending) softmax probabilities.

Not in the reference: its `cumsum` draws N(0, 1) inputs. The scan itself is
the reference's (`x.cumsum(axis=-1)`, kernels/cumsum/kernel.py:12-13)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_cumsum_probs
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="cumsum_probs",
    axon_kernel=kernel_cumsum_probs,
    dim_vars=("m", "n"),
    input_specs=(("probs", ("m", "n")),),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"),
)
