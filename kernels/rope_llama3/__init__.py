"""Spec `rope_llama3`: rotate-half RoPE on token-major q[b, s, hq, d] and
k[b, s, hkv, d] (GQA) with fp32 cos/sin[s, d] from theta = 500000.

Not in the reference, whose `rope` spec is the split d-major layout with
bf16 random-angle cos/sin. The rotation itself is the same: for i < d/2,
out[i] = x[i] cos[i] - x[i + d/2] sin[i] and
out[i + d/2] = x[i + d/2] cos[i + d/2] + x[i] sin[i + d/2]
(kernels/rope/kernel.py:33-36 with x_even = x[..., :d/2], x_odd = x[..., d/2:])."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_rope_llama3
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="rope_llama3",
    axon_kernel=kernel_rope_llama3,
    dim_vars=("b", "s", "hq", "hkv", "d"),
    input_specs=(
        ("q", ("b", "s", "hq", "d")),
        ("k", ("b", "s", "hkv", "d")),
        ("cos", ("s", "d")),
        ("sin", ("s", "d")),
    ),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"),
)
