"""Host-side dtype handling for spec inputs, without `ml_dtypes`.

The reference's spec packages draw float64 numbers from numpy and convert them
with `.astype(ml_dtypes.bfloat16)` (kernels/rmsnorm/refs.py:33-34). That
package is not part of this stack, so a bf16 host array is a CPU
`torch.bfloat16` tensor here. The conversion keeps the same rounding chain as
ml_dtypes' double constructor: float64 -> float32 (round to nearest even),
then float32 -> bfloat16 (round to nearest even).

When `ml_dtypes` *is* importable (a user's own environment), numpy bf16
arrays are accepted everywhere a host array is: `to_torch` reinterprets their
16-bit payload, so both representations feed the same device path.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

try:  # optional: present in the reference's environment, absent in this image
    import ml_dtypes as _ml_dtypes  # type: ignore[import-not-found]
except ImportError:  # pragma: no cover - depends on the image
    _ml_dtypes = None

# The token a spec passes as `dtype=` for bf16 inputs.
bfloat16 = torch.bfloat16
float16 = np.float16
float32 = np.float32

_NAME_TO_DTYPE: dict[str, Any] = {
    "bfloat16": torch.bfloat16,
    "float16": np.dtype(np.float16),
    "float32": np.dtype(np.float32),
}


def resolve(dtype: Any) -> Any:
    """Map a dtype name, numpy dtype, torch dtype or ml_dtypes dtype to the
    canonical token used by `astype` (torch.bfloat16 or a numpy dtype)."""
    if dtype is None:
        return None
    if isinstance(dtype, str):
        if dtype not in _NAME_TO_DTYPE:
            raise ValueError(f"unsupported dtype name {dtype!r}")
        return _NAME_TO_DTYPE[dtype]
    if dtype is torch.bfloat16:
        return dtype
    if isinstance(dtype, torch.dtype):
        return np.dtype(torch.empty((), dtype=dtype).numpy().dtype)
    if _ml_dtypes is not None and np.dtype(dtype) == np.dtype(_ml_dtypes.bfloat16):
        return torch.bfloat16
    return np.dtype(dtype)


def dtype_name(dtype: Any) -> str:
    """The `--dtype` spelling of a dtype token ("bfloat16", "float32", ...)."""
    tok = resolve(dtype)
    if tok is torch.bfloat16:
        return "bfloat16"
    return np.dtype(tok).name


def astype(values: Any, dtype: Any) -> Any:
    """Convert a float64 (or any numeric) numpy array to the host form of
    `dtype`: numpy for float16/float32, a CPU torch tensor for bfloat16."""
    tok = resolve(dtype)
    arr = np.asarray(values)
    if tok is torch.bfloat16:
        f32 = np.ascontiguousarray(arr.astype(np.float32))
        return torch.from_numpy(f32).to(torch.bfloat16)
    return np.ascontiguousarray(arr.astype(tok))


def is_bf16(a: Any) -> bool:
    if isinstance(a, torch.Tensor):
        return a.dtype == torch.bfloat16
    if _ml_dtypes is not None and isinstance(a, np.ndarray):
        return a.dtype == np.dtype(_ml_dtypes.bfloat16)
    return False


def to_torch(a: Any) -> torch.Tensor:
    """A host array (numpy, ml_dtypes numpy bf16 or torch) as a contiguous
    CPU torch tensor of the same element type."""
    if isinstance(a, torch.Tensor):
        return a.contiguous()
    arr = np.ascontiguousarray(np.asarray(a))
    if _ml_dtypes is not None and arr.dtype == np.dtype(_ml_dtypes.bfloat16):
        return torch.from_numpy(arr.view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(arr)


def to_f32_numpy(a: Any) -> np.ndarray:
    """Any host or device array as a float32 numpy array (the fp32 upcast the
    correctness check applies, src/axon/bench_runner.py:562-573)."""
    if isinstance(a, torch.Tensor):
        return a.detach().to("cpu", torch.float32).numpy()
    arr = np.asarray(a)
    if _ml_dtypes is not None and arr.dtype == np.dtype(_ml_dtypes.bfloat16):
        return arr.astype(np.float32)
    return arr.astype(np.float32)


def to_f32_torch(a: Any) -> torch.Tensor:
    """Any host array as an fp32 CPU torch tensor: the coercion the reference's
    harness applies before calling a spec's `torch_ref`
    (src/axon/case_gen.py:190-201)."""
    if isinstance(a, torch.Tensor):
        return a.detach().to("cpu", torch.float32)
    return torch.from_numpy(np.ascontiguousarray(to_f32_numpy(a)))
