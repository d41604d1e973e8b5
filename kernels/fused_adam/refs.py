"""References and inputs for `fused_adam` (kernels/fused_adam/refs.py:21-67).

Update, elementwise, with per-row scalars step_size, inv_bc2_sqrt, wd:
  g  = grad + wd * param
  m' = 0.9 m + (1 - 0.9) g
  v' = 0.999 v + (1 - 0.999) g^2
  p' = p - m' / (sqrt(v') * inv_bc2_sqrt + 1e-8) * step_size
Draw order: param, grad, exp_avg ~ N(0,1); exp_avg_sq = |N(0,1)|; then the
constant (p, 1) fills step_size = 1e-3, inv_bc2_sqrt = 1, wd = 0.01; all in
`dtype` (bf16 by default)."""

import numpy as np
import torch

from axon.dtypes import astype, bfloat16

BETA1 = 0.9
BETA2 = 0.999
EPS = 1e-8
ONE_MINUS_BETA1 = 1.0 - BETA1
ONE_MINUS_BETA2 = 1.0 - BETA2


def baseline_op(param, grad, exp_avg, exp_avg_sq, step_size, inv_bc2_sqrt, wd):
    g = grad + wd * param
    m = BETA1 * exp_avg + ONE_MINUS_BETA1 * g
    v = BETA2 * exp_avg_sq + ONE_MINUS_BETA2 * (g * g)
    denom = np.sqrt(v) * inv_bc2_sqrt + EPS
    return param - m / denom * step_size, m, v


def torch_ref(param, grad, exp_avg, exp_avg_sq, step_size, inv_bc2_sqrt, wd):
    g = grad + wd * param
    m = BETA1 * exp_avg + ONE_MINUS_BETA1 * g
    v = BETA2 * exp_avg_sq + ONE_MINUS_BETA2 * (g * g)
    denom = torch.sqrt(v) * inv_bc2_sqrt + EPS
    return (param - m / denom * step_size, m, v)


def make_inputs(*, p, f, dtype=bfloat16, rng):
    full, col = (p, f), (p, 1)
    return (
        astype(rng.standard_normal(full), dtype),
        astype(rng.standard_normal(full), dtype),
        astype(rng.standard_normal(full), dtype),
        astype(np.abs(rng.standard_normal(full)), dtype),
        astype(np.full(col, 1e-3), dtype),
        astype(np.full(col, 1.0), dtype),
        astype(np.full(col, 0.01), dtype),
    )
