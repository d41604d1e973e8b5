"""Spec `rmsnorm_weighted`: Llama-style RMSNorm, x * rsqrt(mean(x^2) + 1e-6) * w.

Not in the reference: the reference's `rmsnorm` is the sum form without eps
or weight. This package states the mean/eps/weight form with the same spec
layout (dims (m, n), tile args M/N) and one extra input `weight[n]`."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_rmsnorm_weighted
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="rmsnorm_weighted",
    axon_kernel=kernel_rmsnorm_weighted,
    dim_vars=("m", "n"),
    input_specs=(("x", ("m", "n")), ("weight", ("n",))),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"),
)
