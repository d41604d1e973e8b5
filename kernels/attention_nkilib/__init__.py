"""Spec `attention_nkilib`: single-head softmax(q @ k_t) @ v with k given
transposed (d, s), no scale inside and no max subtraction
(kernels/attention_nkilib/__init__.py:22-43 of the reference)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_attention_nkilib
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="attention_nkilib",
    axon_kernel=kernel_attention_nkilib,
    dim_vars=("s", "d"),
    input_specs=(("q", ("s", "d")), ("k_t", ("d", "s")), ("v", ("s", "d"))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K", "TILES_IN_BLOCK_P"),
    tile_options=(1, 2, 4, 8, 16),
)
