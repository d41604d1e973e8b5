"""AxonArray statement of `cumsum_probs`."""

from axon import AxonArray


def kernel_cumsum_probs(probs: AxonArray) -> AxonArray:
    return probs.cumsum(axis=-1)
