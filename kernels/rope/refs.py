"""References and inputs for `rope` (kernels/rope/refs.py:20-46).

Draw order: x_even ~ N(0,1), x_odd ~ N(0,1), then one angle per element
~ U(-pi, pi); cos/sin of that angle. All four converted to `dtype`."""

import numpy as np

from axon.dtypes import astype, bfloat16


def baseline_op(x_even, x_odd, cos, sin):
    return x_even * cos - x_odd * sin, x_odd * cos + x_even * sin


def torch_ref(x_even, x_odd, cos, sin):
    return (x_even * cos - x_odd * sin, x_odd * cos + x_even * sin)


def make_inputs(*, half_d, free, dtype=bfloat16, rng):
    shape = (half_d, free)
    x_even = rng.standard_normal(shape)
    x_odd = rng.standard_normal(shape)
    angle = rng.uniform(-np.pi, np.pi, shape)
    return (
        astype(x_even, dtype),
        astype(x_odd, dtype),
        astype(np.cos(angle), dtype),
        astype(np.sin(angle), dtype),
    )
