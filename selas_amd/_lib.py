"""ctypes binding of libselas_amd.so (the C ABI declared in include/selas_amd.h).

The library is loaded lazily, the first time a kernel is called, so that the
package imports on machines without a GPU. A missing library or a missing GPU
is an error, never a silent fallback: every product path goes through here.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libselas_amd.so"
ABI_VERSION = 6

OK, EINVAL, EUNSUPPORTED, EHIP = 0, 1, 2, 3
F32, F16, BF16 = 0, 1, 2
CODEC_NF4, CODEC_INT8_ROW = 0, 1

DTYPE_CODES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

# Exported symbols and their argument types (c_void_p for pointers, c_int64 for sizes/strides).
_P, _I64, _INT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
_F16x = ctypes.POINTER(ctypes.c_float)
SIGNATURES: dict[str, list] = {
    "selas_nf4_dequant": [_P, _P, _I64, _I64, _F16x, _P, _INT, _P],
    "selas_nf4_encode": [_P, _I64, _I64, _F16x, _P, _P, _P],
    "selas_nf4_linear": [_P, _I64, _I64, _I64, _P, _P, _I64, _F16x, _I64, _P, _P, _I64, _INT, _P, _I64, _P],
    "selas_nf4_linear_grouped": [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _F16x, _INT, _P],
    "selas_nf4_linear_batched": [_P, _I64, _I64, _F16x, _INT, _P, _I64, _P],
    "selas_linear_workspace_bytes": [_P, _I64, _INT, ctypes.POINTER(ctypes.c_int64)],
    "selas_nf4_linear_grouped_static": [_P, _I64, _I64, _I64, _P, _I64, _I64, _F16x, _INT, _P],
    "selas_int8_row_dequant": [_P, _P, _I64, _I64, _P, _INT, _P],
    "selas_int8_row_encode": [_P, _I64, _I64, _P, _P, _P],
    "selas_int8_row_linear": [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _INT, _P, _I64, _P],
    "selas_int8_row_linear_batched": [_P, _I64, _INT, _P, _I64, _P],
    "selas_int8_row_linear_grouped": [_P, _I64, _I64, _I64, _P, _I64, _I64, _INT, _P],
    "selas_mod_in": [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _INT, _P],
    "selas_gated_add": [_P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _INT, _I64, _I64, _INT, _P, _P],
    "selas_gated_add_mod": [_P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _INT, _I64, _I64, _INT, _P, _P, _I64,
                            _P, _P, _INT, _P],
    "selas_qkv_single": [_P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _INT, _P],
    "selas_qkv_double": [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P,
                         _P, _P, _INT, _P],
    "selas_gelu": [_P, _I64, _I64, _I64, _P, _INT, _P],
    "selas_attn_mlp": [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _INT, _P],
    "selas_attention": [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _INT, _P],
    "selas_transpose_heads": [_P, _I64, _I64, _I64, _P, _INT, _P],
}


MAX_BATCHED_LINEARS = 4


class GemmProblem(ctypes.Structure):
    """selas_nf4_gemm_problem (include/selas_amd.h)."""

    _fields_ = [("x", _P), ("M", _I64), ("K", _I64), ("ldx", _I64), ("packed", _P), ("absmax", _P), ("N", _I64),
                ("bias", _P), ("y", _P), ("ldy", _I64), ("y2", _P), ("ldy2", _I64), ("gelu_cols", _I64)]


class GemvDesc(ctypes.Structure):
    """selas_nf4_gemv_desc (include/selas_amd.h): one weight of a grouped skinny launch."""

    _fields_ = [("packed", _P), ("absmax", _P), ("bias", _P), ("y", _P), ("n", _I64), ("ldy", _I64)]


STATIC_MAX_WEIGHTS = 1023
STATIC_MAX_STREAMS = 8


class Unsupported(NotImplementedError):
    """A valid call outside what the fused kernels cover (the caller may use another path)."""


class HipError(RuntimeError):
    """A HIP runtime or launch failure inside the library."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The loaded library (thread-safe, once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m selas_amd.build` "
                                   "(hipcc, gfx950); selas_amd has no CPU fallback")
            lib = ctypes.CDLL(str(LIB_PATH))
            lib.selas_last_error.restype = ctypes.c_char_p
            lib.selas_last_error.argtypes = []
            lib.selas_abi_version.restype = ctypes.c_int
            lib.selas_abi_version.argtypes = []
            if lib.selas_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI {lib.selas_abi_version()}, expected {ABI_VERSION}: rebuild it")
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = ctypes.c_int
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Calls an entry point and turns its status into the reference's exception types."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc == OK:
        return
    msg = lib.selas_last_error().decode(errors="replace")
    if rc == EINVAL:
        raise ValueError(msg)
    if rc == EUNSUPPORTED:
        raise Unsupported(msg)
    raise HipError(msg)


_ws_sizes: dict[tuple, int] = {}


def workspace_bytes(codec: int, shapes, device: torch.device) -> int:
    """Bytes of scratch a tiled linear launch over problems of these (M, K, N) shapes needs on ``device``
    (selas_linear_workspace_bytes; 0 for most shapes). The answer depends on the shapes and the GPU's CU
    count only, so it is kept per (device, codec, shapes)."""
    key = (device.index, codec, tuple(shapes))
    n = _ws_sizes.get(key)
    if n is None:
        arr = (GemmProblem * max(len(shapes), 1))()
        for i, (m, k, nn) in enumerate(shapes):
            arr[i].M, arr[i].K, arr[i].N = m, k, nn
        out = ctypes.c_int64(0)
        with torch.cuda.device(device):
            call("selas_linear_workspace_bytes", ctypes.addressof(arr), len(shapes), codec, ctypes.byref(out))
        n = _ws_sizes[key] = int(out.value)
    return n


def workspace(codec: int, shapes, device: torch.device) -> tuple[torch.Tensor | None, int]:
    """(scratch tensor or None, its size in bytes) for a tiled linear launch: allocated from torch's caching
    allocator on the current stream, per call, so stream-ordered reuse keeps it private to the launch."""
    n = workspace_bytes(codec, shapes, device)
    if n == 0:
        return None, 0
    return torch.empty(n, dtype=torch.uint8, device=device), n


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (kernels must run on it)."""
    return torch.cuda.current_stream(device).cuda_stream


def code_array(code) -> ctypes.Array:
    vals = [float(c) for c in code]
    if len(vals) != 16:
        raise ValueError(f"nf4 codebook needs 16 entries, got {len(vals)}")
    return (ctypes.c_float * 16)(*vals)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}") from None


def require_gpu(*ts: torch.Tensor) -> torch.device:
    """All tensors on one GPU; returns it. CPU tensors are an error: there is no CPU path."""
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"selas_amd runs on the GPU; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev
