"""ctypes binding of libaxon_hip.so (the C ABI in include/axon_hip.h).

This module is the only way device work reaches the GPU: it loads the
in-tree library and raises `HipLibraryError` when the library is missing or a
call fails; there is no CPU or torch fallback anywhere behind it. torch is
used for device memory and the current stream only.

The host-only entry points (names, manifests, legality checks, output
descriptors) never touch the HIP runtime, so they work on machines without a
GPU.
"""

from __future__ import annotations

import ctypes
import json
import threading
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Sequence

from enzyme_amd.candidate_filter import TileConstraint

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libaxon_hip.so"

AXON_OK = 0
AXON_EINVAL = 1
AXON_ENOKERNEL = 2
AXON_EDTYPE = 3
AXON_EARG = 4
AXON_EWORKSPACE = 5
AXON_EHIP = 6
AXON_EBUFFER = 7

AXON_BF16 = 0
AXON_F16 = 1
AXON_F32 = 2

_STATUS_NAMES = {
    AXON_EINVAL: "AXON_EINVAL",
    AXON_ENOKERNEL: "AXON_ENOKERNEL",
    AXON_EDTYPE: "AXON_EDTYPE",
    AXON_EARG: "AXON_EARG",
    AXON_EWORKSPACE: "AXON_EWORKSPACE",
    AXON_EHIP: "AXON_EHIP",
    AXON_EBUFFER: "AXON_EBUFFER",
}

# Every symbol include/axon_hip.h declares.
EXPORTED_SYMBOLS = (
    "axon_abi_version",
    "axon_last_error",
    "axon_kernel_count",
    "axon_kernel_name",
    "axon_kernel_variants",
    "axon_variant_describe",
    "axon_variant_manifest",
    "axon_variant_outputs",
    "axon_variant_check",
    "axon_variant_workspace",
    "axon_variant_launch",
    "axon_variant_launch_noalloc",
    "axon_copy",
    "axon_copy_shape",
    "axon_scan_poll_bound",
)


class HipLibraryError(RuntimeError):
    """The native library is missing, or a native call returned an error."""

    def __init__(self, message: str, status: int | None = None):
        super().__init__(message)
        self.status = status


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_voidpp = ctypes.POINTER(ctypes.c_void_p)


def _declare(lib: ctypes.CDLL) -> None:
    sig = {
        "axon_abi_version": (ctypes.c_int, []),
        "axon_last_error": (ctypes.c_char_p, []),
        "axon_kernel_count": (ctypes.c_int, []),
        "axon_kernel_name": (ctypes.c_char_p, [ctypes.c_int]),
        "axon_kernel_variants": (ctypes.c_int, [ctypes.c_char_p]),
        "axon_variant_describe": (
            ctypes.c_int,
            [ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t],
        ),
        "axon_variant_manifest": (
            ctypes.c_int,
            [ctypes.c_char_p, ctypes.c_int, _i64p, ctypes.c_int, ctypes.c_int,
             ctypes.c_char_p, ctypes.c_size_t],
        ),
        "axon_variant_outputs": (
            ctypes.c_int,
            [ctypes.c_char_p, _i64p, ctypes.c_int, _i32p, ctypes.c_int, ctypes.c_int,
             _i64p, _i32p, _i32p, ctypes.c_int],
        ),
        "axon_variant_check": (
            ctypes.c_int,
            [ctypes.c_char_p, ctypes.c_int, _i32p, ctypes.c_int, _i64p, ctypes.c_int,
             _i32p, ctypes.c_int],
        ),
        "axon_variant_workspace": (
            ctypes.c_size_t,
            [ctypes.c_char_p, ctypes.c_int, _i32p, ctypes.c_int, _i64p, ctypes.c_int,
             _i32p, ctypes.c_int],
        ),
        "axon_variant_launch": (
            ctypes.c_int,
            [ctypes.c_char_p, ctypes.c_int, _i32p, ctypes.c_int, _i64p, ctypes.c_int,
             _i32p, ctypes.c_int, _voidpp, ctypes.c_int, _voidpp, ctypes.c_int,
             ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
        ),
        "axon_variant_launch_noalloc": (
            ctypes.c_int,
            [ctypes.c_char_p, ctypes.c_int, _i32p, ctypes.c_int, _i64p, ctypes.c_int,
             _i32p, ctypes.c_int, _voidpp, ctypes.c_int, _voidpp, ctypes.c_int,
             ctypes.c_void_p],
        ),
        "axon_copy": (
            ctypes.c_int,
            [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
        ),
        "axon_copy_shape": (
            ctypes.c_int,
            [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p],
        ),
        "axon_scan_poll_bound": (ctypes.c_uint32, [ctypes.c_uint32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def lib() -> ctypes.CDLL:
    """The loaded library; raises HipLibraryError if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.is_file():
                raise HipLibraryError(
                    f"native library {LIB_PATH} is missing: build it with "
                    "`python -m enzyme_amd.build` (hipcc, gfx950)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            _declare(handle)
            if handle.axon_abi_version() != 1:
                raise HipLibraryError("libaxon_hip.so ABI version mismatch")
            _lib = handle
        return _lib


def last_error() -> str:
    msg = lib().axon_last_error()
    return msg.decode() if msg else ""


def _raise(status: int, what: str) -> None:
    name = _STATUS_NAMES.get(status, str(status))
    raise HipLibraryError(f"{what} failed with {name}: {last_error()}", status)


def _arr(ctype, values: Sequence[int]):
    arr = (ctype * max(1, len(values)))(*[int(v) for v in values])
    return arr


# ---------------------------------------------------------------------------
# host-only queries
# ---------------------------------------------------------------------------
def kernel_names() -> list[str]:
    h = lib()
    return [h.axon_kernel_name(i).decode() for i in range(h.axon_kernel_count())]


def variant_count(kernel: str) -> int:
    return int(lib().axon_kernel_variants(kernel.encode()))


def describe(kernel: str, hw_variant: int) -> dict[str, Any]:
    buf = ctypes.create_string_buffer(4096)
    rc = lib().axon_variant_describe(kernel.encode(), hw_variant, buf, len(buf))
    if rc != AXON_OK:
        _raise(rc, f"describe({kernel}, v{hw_variant})")
    return json.loads(buf.value.decode())


def manifest(kernel: str, hw_variant: int, dims: Sequence[int], dtype: int) -> tuple[TileConstraint, ...]:
    buf = ctypes.create_string_buffer(4096)
    d = _arr(ctypes.c_int64, dims)
    rc = lib().axon_variant_manifest(kernel.encode(), hw_variant, d, len(dims), dtype, buf, len(buf))
    if rc != AXON_OK:
        _raise(rc, f"manifest({kernel}, v{hw_variant})")
    value = json.loads(buf.value.decode())
    return tuple(TileConstraint(**rec) for rec in value["constraints"])


@dataclass(frozen=True)
class OutputDesc:
    shape: tuple[int, ...]
    dtype: int


def outputs(kernel: str, dims: Sequence[int], dtypes: Sequence[int]) -> list[OutputDesc]:
    max_rank, cap = 6, 8
    shapes = (ctypes.c_int64 * (max_rank * cap))()
    ranks = (ctypes.c_int32 * cap)()
    odt = (ctypes.c_int32 * cap)()
    n = lib().axon_variant_outputs(
        kernel.encode(), _arr(ctypes.c_int64, dims), len(dims), _arr(ctypes.c_int32, dtypes),
        len(dtypes), max_rank, shapes, ranks, odt, cap,
    )
    if n < 0:
        _raise(-n, f"outputs({kernel})")
    return [
        OutputDesc(tuple(shapes[i * max_rank + k] for k in range(ranks[i])), int(odt[i]))
        for i in range(n)
    ]


def check(
    kernel: str, hw_variant: int, tiles: Sequence[int], dims: Sequence[int], dtypes: Sequence[int]
) -> tuple[int, str]:
    """(status, reason): status AXON_OK when the tile tuple is legal."""
    rc = lib().axon_variant_check(
        kernel.encode(), hw_variant, _arr(ctypes.c_int32, tiles), len(tiles),
        _arr(ctypes.c_int64, dims), len(dims), _arr(ctypes.c_int32, dtypes), len(dtypes),
    )
    return int(rc), ("" if rc == AXON_OK else last_error())


def workspace_bytes(
    kernel: str, hw_variant: int, tiles: Sequence[int], dims: Sequence[int], dtypes: Sequence[int]
) -> int:
    return int(
        lib().axon_variant_workspace(
            kernel.encode(), hw_variant, _arr(ctypes.c_int32, tiles), len(tiles),
            _arr(ctypes.c_int64, dims), len(dims), _arr(ctypes.c_int32, dtypes), len(dtypes),
        )
    )


# ---------------------------------------------------------------------------
# device side (torch tensors for memory, torch's current stream)
# ---------------------------------------------------------------------------
def _torch():
    import torch

    return torch


def dtype_code(t) -> int:
    torch = _torch()
    table = {torch.bfloat16: AXON_BF16, torch.float16: AXON_F16, torch.float32: AXON_F32}
    if t.dtype not in table:
        raise HipLibraryError(f"unsupported tensor dtype {t.dtype}")
    return table[t.dtype]


def torch_dtype(code: int):
    torch = _torch()
    return {AXON_BF16: torch.bfloat16, AXON_F16: torch.float16, AXON_F32: torch.float32}[code]


class Launcher:
    """One resolved (kernel, hw_variant, tiles, dims, dtypes) key with its
    outputs and workspace preallocated, ready to be enqueued repeatedly."""

    def __init__(
        self,
        kernel: str,
        hw_variant: int,
        tiles: Sequence[int],
        dims: Sequence[int],
        inputs: Sequence[Any],
        input_shapes: Sequence[tuple[int, ...]] | None = None,
        outputs_: Sequence[Any] | None = None,
        noalloc: bool = False,
    ):
        """`noalloc=True` launches through axon_variant_launch_noalloc: no
        workspace is allocated here, the library's static per-GPU array
        serves as the kernels' workspace."""
        torch = _torch()
        self.noalloc = bool(noalloc)
        self.kernel = kernel
        self.hw_variant = int(hw_variant)
        self.tiles = [int(t) for t in tiles]
        self.dims = [int(d) for d in dims]
        if not inputs:
            raise HipLibraryError(f"{kernel}: no inputs")
        device = inputs[0].device
        if device.type != "cuda":
            raise HipLibraryError(f"{kernel}: inputs must be GPU tensors, got {device}")
        for i, t in enumerate(inputs):
            if not isinstance(t, torch.Tensor) or t.device != device:
                raise HipLibraryError(f"{kernel}: input {i} is not a tensor on {device}")
            if not t.is_contiguous():
                raise HipLibraryError(f"{kernel}: input {i} is not contiguous")
            if input_shapes is not None and tuple(t.shape) != tuple(input_shapes[i]):
                raise HipLibraryError(
                    f"{kernel}: input {i} has shape {tuple(t.shape)}, spec needs {tuple(input_shapes[i])}"
                )
        self.inputs = list(inputs)
        self.dtypes = [dtype_code(t) for t in inputs]
        status, why = check(kernel, self.hw_variant, self.tiles, self.dims, self.dtypes)
        if status != AXON_OK:
            raise HipLibraryError(f"{kernel} v{hw_variant} tiles {self.tiles}: {why}", status)
        descs = outputs(kernel, self.dims, self.dtypes)
        if outputs_ is None:
            self.outputs = [
                torch.empty(d.shape, dtype=torch_dtype(d.dtype), device=device) for d in descs
            ]
        else:
            if len(outputs_) != len(descs):
                raise HipLibraryError(f"{kernel}: {len(descs)} outputs needed")
            for i, (t, d) in enumerate(zip(outputs_, descs)):
                if tuple(t.shape) != d.shape or dtype_code(t) != d.dtype or not t.is_contiguous():
                    raise HipLibraryError(f"{kernel}: output {i} must be contiguous {d.shape}")
            self.outputs = list(outputs_)
        ws = 0 if self.noalloc else workspace_bytes(kernel, self.hw_variant, self.tiles, self.dims,
                                                    self.dtypes)
        # A caller workspace starts zero-filled (every launch leaves it ready
        # for the next one).
        self.workspace = torch.zeros(ws, dtype=torch.uint8, device=device) if ws else None
        self._pack()

    def _pack(self) -> None:
        self._c_kernel = self.kernel.encode()
        self._c_tiles = _arr(ctypes.c_int32, self.tiles)
        self._c_dims = _arr(ctypes.c_int64, self.dims)
        self._c_dtypes = _arr(ctypes.c_int32, self.dtypes)
        self._c_in = (ctypes.c_void_p * len(self.inputs))(*[t.data_ptr() for t in self.inputs])
        self._c_out = (ctypes.c_void_p * len(self.outputs))(*[t.data_ptr() for t in self.outputs])
        self._c_ws = self.workspace.data_ptr() if self.workspace is not None else None
        self._c_ws_bytes = self.workspace.numel() if self.workspace is not None else 0

    def rebind(self, inputs: Sequence[Any], outputs_: Sequence[Any]) -> None:
        """Point the launch at another buffer set of identical shapes/dtypes."""
        for a, b in zip(inputs, self.inputs):
            if a.shape != b.shape or a.dtype != b.dtype or a.device != b.device or not a.is_contiguous():
                raise HipLibraryError(f"{self.kernel}: rebind input mismatch")
        for a, b in zip(outputs_, self.outputs):
            if a.shape != b.shape or a.dtype != b.dtype or a.device != b.device or not a.is_contiguous():
                raise HipLibraryError(f"{self.kernel}: rebind output mismatch")
        self.inputs = list(inputs)
        self.outputs = list(outputs_)
        self._pack()

    def launch(self, stream: Any = None) -> None:
        torch = _torch()
        s = stream if stream is not None else torch.cuda.current_stream(self.inputs[0].device)
        if self.noalloc:
            rc = lib().axon_variant_launch_noalloc(
                self._c_kernel, self.hw_variant, self._c_tiles, len(self.tiles), self._c_dims,
                len(self.dims), self._c_dtypes, len(self.dtypes), self._c_in, len(self.inputs),
                self._c_out, len(self.outputs), ctypes.c_void_p(s.cuda_stream),
            )
        else:
            rc = lib().axon_variant_launch(
                self._c_kernel, self.hw_variant, self._c_tiles, len(self.tiles), self._c_dims,
                len(self.dims), self._c_dtypes, len(self.dtypes), self._c_in, len(self.inputs),
                self._c_out, len(self.outputs), self._c_ws, self._c_ws_bytes,
                ctypes.c_void_p(s.cuda_stream),
            )
        if rc != AXON_OK:
            _raise(rc, f"launch({self.kernel}, v{self.hw_variant}, tiles {self.tiles})")


def run(kernel: str, hw_variant: int, tiles: Sequence[int], dims: Sequence[int], *inputs: Any):
    """Allocate outputs, launch once on the current stream, return the outputs
    (a single tensor when the kernel has one output)."""
    ln = Launcher(kernel, hw_variant, tiles, dims, inputs)
    ln.launch()
    return ln.outputs[0] if len(ln.outputs) == 1 else tuple(ln.outputs)


def run_variant(meta: dict[str, Any], inputs: Sequence[Any], tiles: Sequence[int]):
    """Entry used by emitted variant modules: launch the module's family and
    variant with `tiles` on `inputs` (GPU tensors in the spec's shapes)."""
    shapes = meta.get("input_shapes")
    ln = Launcher(
        meta["kernel"], meta["hw_variant"], tiles, meta["dims"], list(inputs),
        input_shapes=[tuple(s) for s in shapes] if shapes is not None else None,
    )
    ln.launch()
    return ln.outputs[0] if len(ln.outputs) == 1 else tuple(ln.outputs)


def scan_poll_bound(polls: int) -> int:
    """Set the single-pass cumsum poll bound (0 = always recompute earlier
    chunk totals from the input); returns the previous bound."""
    return int(lib().axon_scan_poll_bound(int(polls)))


COPY_SHAPES = {
    0: "one 16-byte vector per thread, grid-stride over <= 16384 blocks of 256",
    1: "one-shot, 8 vectors per thread",
    2: "one-shot, 4 vectors per thread",
    3: "one 16-byte vector per thread, grid-stride over 1024 blocks of 256",
}


def copy(src, dst, shape: int = 0) -> None:
    """Plain device copy (the traffic-counter calibration kernel) in one of
    the launch shapes of COPY_SHAPES."""
    torch = _torch()
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise HipLibraryError("copy: size mismatch")
    s = torch.cuda.current_stream(src.device)
    rc = lib().axon_copy_shape(
        ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), nbytes, int(shape),
        ctypes.c_void_p(s.cuda_stream),
    )
    if rc != AXON_OK:
        _raise(rc, "axon_copy_shape")
