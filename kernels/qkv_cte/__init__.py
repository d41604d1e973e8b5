"""Spec `qkv_cte`: the QKV context-encoding projection core, residual add ->
RMSNorm (mean form, eps 1e-6, no gamma) -> projection,
    h = x + mlp_prev + attention_prev;  out = (h / sqrt(mean(h^2) + eps)) @ w,
with the reference's dims, input names and order (kernels/qkv_cte/__init__.py:23-37
of the reference; M = tokens, K = hidden, N = fused QKV width)."""

from axon.kernel_spec import KernelSpec

from .kernel import kernel_qkv_cte
from .refs import baseline_op, make_inputs, torch_ref

SPEC = KernelSpec(
    name="qkv_cte",
    axon_kernel=kernel_qkv_cte,
    dim_vars=("m", "n", "k"),
    input_specs=(
        ("x", ("m", "k")),
        ("mlp_prev", ("m", "k")),
        ("attention_prev", ("m", "k")),
        ("w", ("k", "n")),
    ),
    baseline_op=baseline_op,
    torch_ref=torch_ref,
    make_inputs=make_inputs,
    tile_args=("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K"),
)
