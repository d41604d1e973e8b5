"""An eager, torch-backed `AxonArray`.

The reference's `AxonArray` (src/axon/ir.py:27-160) records a graph for its
synthesizer. Synthesis is not part of this backend, but every spec's
`kernel.py` imports `AxonArray` and is written against its operator surface,
so this class keeps exactly that surface (`+ - * / @`, `sum(axis,
keep_dims)`, `sqrt`, `exp`, `transpose`, `relu`, `silu`, `softmax`, `cumsum`,
`broadcast_like`, `.shape`) and evaluates it eagerly in float64 on the CPU.

That gives each spec a third, independent statement of its math: the tests
run `kernel.py` through this class and compare it with the spec's `torch_ref`
and `baseline_op`, which catches a `kernel.py` / `refs.py` drift (the
reference hit one, kernels/rmsnorm_matmul/refs.py:17-20).
"""

from __future__ import annotations

from typing import Any

import torch

from enzyme_amd.dtypes import to_f32_torch


class AxonArray:
    __slots__ = ("value",)

    def __init__(self, value: Any):
        if isinstance(value, AxonArray):
            value = value.value
        if not isinstance(value, torch.Tensor):
            value = to_f32_torch(value)
        self.value = value.to(torch.float64)

    # -- shape -----------------------------------------------------------
    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(int(d) for d in self.value.shape)

    # -- binary ops --------------------------------------------------------
    @staticmethod
    def _v(other: Any) -> Any:
        return other.value if isinstance(other, AxonArray) else other

    def __add__(self, other: Any) -> AxonArray:
        return AxonArray(self.value + self._v(other))

    __radd__ = __add__

    def __sub__(self, other: Any) -> AxonArray:
        return AxonArray(self.value - self._v(other))

    def __rsub__(self, other: Any) -> AxonArray:
        return AxonArray(self._v(other) - self.value)

    def __mul__(self, other: Any) -> AxonArray:
        return AxonArray(self.value * self._v(other))

    __rmul__ = __mul__

    def __truediv__(self, other: Any) -> AxonArray:
        return AxonArray(self.value / self._v(other))

    def __matmul__(self, other: Any) -> AxonArray:
        if not isinstance(other, AxonArray):
            raise TypeError("matmul expects AxonArray operand")
        if self.value.dim() != 2 or other.value.dim() != 2:
            raise ValueError("matmul expects rank-2 inputs")
        return AxonArray(self.value @ other.value)

    # -- reductions / unary ops ------------------------------------------
    def sum(self, axis: Any = None, keep_dims: bool = False) -> AxonArray:
        if axis is None:
            out = self.value.sum()
            if keep_dims:
                out = out.reshape([1] * self.value.dim())
            return AxonArray(out)
        return AxonArray(self.value.sum(dim=axis, keepdim=keep_dims))

    def broadcast_like(self, other: AxonArray) -> AxonArray:
        return AxonArray(self.value.expand_as(other.value).clone())

    def sqrt(self) -> AxonArray:
        return AxonArray(torch.sqrt(self.value))

    def exp(self) -> AxonArray:
        return AxonArray(torch.exp(self.value))

    def transpose(self) -> AxonArray:
        if self.value.dim() == 2:
            return AxonArray(self.value.t().contiguous())
        return AxonArray(self.value)

    def relu(self) -> AxonArray:
        return AxonArray(torch.relu(self.value))

    def silu(self) -> AxonArray:
        v = self.value
        return AxonArray(v / (1.0 + torch.exp(-v)))

    def softmax(self, axis: int = -1) -> AxonArray:
        return AxonArray(torch.softmax(self.value, dim=axis))

    def cumsum(self, axis: int = -1) -> AxonArray:
        return AxonArray(torch.cumsum(self.value, dim=axis))

    # -- extensions beyond the reference surface --------------------------
    # Needed to state the token-major RoPE and the multi-head causal
    # attention specs; the reference's rank-2 specs never use them.
    def __getitem__(self, index: Any) -> AxonArray:
        return AxonArray(self.value[index])

    def reshape(self, shape: tuple[int, ...]) -> AxonArray:
        return AxonArray(self.value.reshape(shape))

    @staticmethod
    def concat(parts: list[AxonArray], axis: int = -1) -> AxonArray:
        return AxonArray(torch.cat([p.value for p in parts], dim=axis))

    def bmm(self, other: AxonArray) -> AxonArray:
        """Matrix product over the last two axes, batched over the rest."""
        return AxonArray(torch.matmul(self.value, other.value))

    def transpose_last(self) -> AxonArray:
        return AxonArray(self.value.transpose(-1, -2).contiguous())

    def causal_mask(self) -> AxonArray:
        """-inf where the key index (last axis) exceeds the query index."""
        s_q, s_k = self.value.shape[-2], self.value.shape[-1]
        mask = torch.ones(s_q, s_k, dtype=torch.bool).triu(1)
        return AxonArray(self.value.masked_fill(mask, float("-inf")))


def evaluate(kernel_fn, *inputs: Any) -> tuple[torch.Tensor, ...]:
    """Run a spec's `axon_kernel` eagerly; always returns a tuple of float64
    tensors (one per kernel output)."""
    out = kernel_fn(*[AxonArray(a) for a in inputs])
    outs = out if isinstance(out, tuple) else (out,)
    return tuple(o.value for o in outs)
