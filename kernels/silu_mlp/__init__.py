"""Spec `silu_mlp`: (silu(x @ w1) * (x @ w2)) @ w3
(kernels/silu_mlp/__init__.py:16-34 of the reference). The reference
package has no `torch_ref`; this one adds it with the same math."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_silu_mlp_full
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="silu_mlp",
    axon_kernel=kernel_silu_mlp_full,
    dim_vars=("m", "n", "k", "p"),
    input_specs=(
        ("x", ("m", "k")),
        ("w1", ("k", "n")),
        ("w2", ("k", "n")),
        ("w3", ("n", "p")),
    ),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K", "TILES_IN_BLOCK_P"),
)
