"""Spec `attention_causal`: multi-head causal attention,
softmax(q k^T / sqrt(d) + causal mask) v with an fp32 softmax, on
[b, h, s, d] tensors.

Not in the reference, whose `attention_nkilib` is single-head, unscaled,
unmasked and without max subtraction; the two matrix products and the
row softmax are the same operations."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_attention_causal
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="attention_causal",
    axon_kernel=kernel_attention_causal,
    dim_vars=("b", "h", "s", "d"),
    input_specs=(("q", ("b", "h", "s", "d")), ("k", ("b", "h", "s", "d")), ("v", ("b", "h", "s", "d"))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K", "TILES_IN_BLOCK_P"),
    tile_options=(1, 2, 4, 8, 16),
)
