"""AxonArray statement of `rope_llama3` (uses the slicing/reshape/concat
extensions of this backend's AxonArray)."""

from axon import AxonArray


def _rotate(x: AxonArray, cos: AxonArray, sin: AxonArray) -> AxonArray:
    half = x.shape[-1] // 2
    c = cos.reshape((1, cos.shape[0], 1, cos.shape[1]))
    s = sin.reshape((1, sin.shape[0], 1, sin.shape[1]))
    rot = AxonArray.concat([x[..., half:] * -1.0, x[..., :half]], axis=-1)
    return x * c + rot * s


def kernel_rope_llama3(q: AxonArray, k: AxonArray, cos: AxonArray, sin: AxonArray):
    return (_rotate(q, cos, sin), _rotate(k, cos, sin))
