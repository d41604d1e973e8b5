"""Spec `rmsnorm_matmul_eps`: (x * rsqrt(mean x^2 + 1e-6)) @ w, the eps form
of `rmsnorm_matmul` (the reference states this form inside
kernels/qkv_cte/kernel.py:25-27), with operands drawn from N(0, 0.02^2)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_rmsnorm_matmul_eps
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="rmsnorm_matmul_eps",
    axon_kernel=kernel_rmsnorm_matmul_eps,
    dim_vars=("m", "n", "k"),
    input_specs=(("x", ("m", "k")), ("w", ("k", "n"))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K"),
)
