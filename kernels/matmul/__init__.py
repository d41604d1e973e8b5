"""Spec `matmul`: x[m, k] @ w[k, n] (the reference's kernels/matmul/__init__.py:13-25,
math in kernels/matmul/kernel.py:7-8)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_matmul
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="matmul",
    axon_kernel=kernel_matmul,
    dim_vars=("m", "n", "k"),
    input_specs=(("x", ("m", "k")), ("w", ("k", "n"))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K"),
)
