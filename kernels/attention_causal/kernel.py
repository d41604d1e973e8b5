"""AxonArray statement of `attention_causal` (uses the batched-matmul,
transpose-last-two, causal-mask and max-shifted softmax of this backend's
eager AxonArray)."""

from axon import AxonArray


def kernel_attention_causal(q: AxonArray, k: AxonArray, v: AxonArray) -> AxonArray:
    d = q.shape[-1]
    scores = q.bmm(k.transpose_last()) * (1.0 / d**0.5)
    return scores.causal_mask().softmax(axis=-1).bmm(v)
