"""AxonArray statement of `attention_nkilib` (kernels/attention_nkilib/kernel.py:14-21)."""

from axon import AxonArray


def kernel_attention_nkilib(q: AxonArray, k_t: AxonArray, v: AxonArray) -> AxonArray:
    e = (q @ k_t).exp()
    return (e / e.sum(axis=1, keep_dims=True)) @ v
