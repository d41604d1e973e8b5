"""Spec `fused_adam`: Adam with L2 weight decay, no AMSGrad; three (p, 1)
per-row scalars broadcast over the free axis
(kernels/fused_adam/__init__.py:27-48 of the reference)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_fused_adam
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="fused_adam",
    axon_kernel=kernel_fused_adam,
    dim_vars=("p", "f"),
    input_specs=(
        ("param", ("p", "f")),
        ("grad", ("p", "f")),
        ("exp_avg", ("p", "f")),
        ("exp_avg_sq", ("p", "f")),
        ("step_size", ("p", 1)),
        ("inv_bc2_sqrt", ("p", 1)),
        ("wd", ("p", 1)),
    ),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N"),
)
