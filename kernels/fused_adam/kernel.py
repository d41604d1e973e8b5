"""AxonArray statement of `fused_adam` (kernels/fused_adam/kernel.py:20-45)."""

from axon import AxonArray

BETA1 = 0.9
BETA2 = 0.999
EPS = 1e-8
ONE_MINUS_BETA1 = 1.0 - BETA1
ONE_MINUS_BETA2 = 1.0 - BETA2


def kernel_fused_adam(param, grad, exp_avg, exp_avg_sq, step_size, inv_bc2_sqrt, wd):
    g = grad + wd * param
    m = BETA1 * exp_avg + ONE_MINUS_BETA1 * g
    v = BETA2 * exp_avg_sq + ONE_MINUS_BETA2 * (g * g)
    denom = v.sqrt() * inv_bc2_sqrt + EPS
    return (param - m / denom * step_size, m, v)
