"""AxonArray statement of `matmul_std002`."""

from axon import AxonArray


def kernel_matmul_std002(a: AxonArray, b: AxonArray) -> AxonArray:
    return a @ b
