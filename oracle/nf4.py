"""NF4 codec oracle (numpy, plus the C restatement in nf4_ref.c): test infrastructure only.

Restates selas/codecs.py:
  * ``decode``  — nf4_dequant_torch (codecs.py:178-199): value = code[nibble] *
    absmax[byte // (blocksize/2)] in fp32, element 2i from the high nibble of
    byte i, then one rounding to the output type.
  * ``encode``  — encode_nf4 (codecs.py:99-119): per-block absmax over the
    flattened tensor, x / absmax (absmax 0 -> 1) in fp32, code index =
    torch.bucketize(x, mids, right=False) with mids = (c[1:] + c[:-1]) / 2 in
    fp32 (ties go to the lower code), packed two per byte, first element high.
  * ``bf16_bits`` / ``f16_bits`` — the fp32 roundings torch applies in
    ``.to(bfloat16)`` / ``.to(float16)`` (round to nearest even).

Pinned by (tests/test_oracle_nf4.py): the reference's packing KAT
(test_codecs.py:47-51), the nearest-code invariant with brute force over all
16 codes (test_codecs.py:66-75), exact decodes with power-of-two absmax, the
midpoint tie rule, the relative-error bound (test_codecs.py:62-63), agreement
of the numpy and C restatements, and the roundings against torch's own casts.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)

F32, F16, BF16 = 0, 1, 2

# --------------------------------------------------------------------------- roundings


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even; NaN -> 0x7FC0."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> IEEE fp16 bit patterns, round to nearest even."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def round_to(x: np.ndarray, out: int) -> np.ndarray:
    """fp32 values rounded to the output type, as stored bits (uint16) or fp32."""
    if out == F32:
        return np.asarray(x, dtype=np.float32)
    return f16_bits(x) if out == F16 else bf16_bits(x)


# --------------------------------------------------------------------------- codec


def decode(packed: np.ndarray, absmax: np.ndarray, blocksize: int, code=NF4_CODE, out: int = F32) -> np.ndarray:
    """Reference NF4 decode of the flattened tensor (see module docstring)."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    absmax = np.asarray(absmax, dtype=np.float32).reshape(-1)
    c = np.asarray(code, dtype=np.float32)
    bpb = blocksize // 2
    a = absmax[np.arange(packed.size) // bpb]
    vals = np.empty(packed.size * 2, dtype=np.float32)
    vals[0::2] = c[packed >> 4] * a
    vals[1::2] = c[packed & 15] * a
    return round_to(vals, out)


def midpoints(code=NF4_CODE) -> np.ndarray:
    c = np.asarray(code, dtype=np.float32)
    return ((c[1:] + c[:-1]) / np.float32(2)).astype(np.float32)


def encode(w: np.ndarray, blocksize: int = 64, code=NF4_CODE) -> tuple[np.ndarray, np.ndarray]:
    """Reference NF4 encode: (packed uint8 [n/2], absmax fp32 [n/blocksize])."""
    flat = np.asarray(w, dtype=np.float32).reshape(-1)
    n = flat.size
    if blocksize <= 0 or n % blocksize or blocksize % 2:
        raise ValueError(f"nf4 needs numel divisible by blocksize ({n} % {blocksize})")
    blocks = flat.reshape(-1, blocksize)
    with np.errstate(invalid="ignore"):
        absmax = np.abs(blocks).max(axis=1).astype(np.float32)
        safe = np.where(absmax > 0, absmax, np.float32(1)).astype(np.float32)
        normed = (blocks / safe[:, None]).reshape(-1).astype(np.float32)
    # bucketize(right=False) == searchsorted(side='left'): count of midpoints < x (NaN sorts last -> 15)
    idx = np.searchsorted(midpoints(code), normed, side="left").astype(np.uint8)
    packed = ((idx[0::2] << 4) | idx[1::2]).astype(np.uint8)
    return packed, absmax


# --------------------------------------------------------------------------- C restatement

_C = {"lib": None}
C_LIB = Path(__file__).resolve().parent / "_build" / "libnf4_oracle.so"


def c_lib():
    """The compiled C restatement (oracle/_build/libnf4_oracle.so), or None if it is not built."""
    if _C["lib"] is None and C_LIB.exists():
        lib = ctypes.CDLL(str(C_LIB))
        lib.nf4o_decode.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_int]
        lib.nf4o_decode.restype = None
        lib.nf4o_encode.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p]
        lib.nf4o_encode.restype = ctypes.c_int
        lib.nf4o_f16_bits.argtypes = [ctypes.c_float]
        lib.nf4o_f16_bits.restype = ctypes.c_uint16
        _C["lib"] = lib
    return _C["lib"]


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def c_decode(packed: np.ndarray, absmax: np.ndarray, blocksize: int, code=NF4_CODE, out: int = F32) -> np.ndarray:
    lib = c_lib()
    if lib is None:
        raise RuntimeError(f"{C_LIB} is not built (make -C oracle)")
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    absmax = np.ascontiguousarray(absmax, dtype=np.float32).reshape(-1)
    c = np.ascontiguousarray(code, dtype=np.float32)
    res = np.empty(packed.size * 2, dtype=np.float32 if out == F32 else np.uint16)
    lib.nf4o_decode(_p(packed), _p(absmax), packed.size, blocksize, _p(c), _p(res), out)
    return res


def c_encode(w: np.ndarray, blocksize: int = 64, code=NF4_CODE) -> tuple[np.ndarray, np.ndarray]:
    lib = c_lib()
    if lib is None:
        raise RuntimeError(f"{C_LIB} is not built (make -C oracle)")
    flat = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    c = np.ascontiguousarray(code, dtype=np.float32)
    packed = np.empty(flat.size // 2, dtype=np.uint8)
    absmax = np.empty(flat.size // blocksize, dtype=np.float32)
    if lib.nf4o_encode(_p(flat), flat.size, blocksize, _p(c), _p(packed), _p(absmax)):
        raise ValueError(f"nf4 needs numel divisible by blocksize ({flat.size} % {blocksize})")
    return packed, absmax


# --------------------------------------------------------------------------- torch restatement (CPU baseline)


def decode_torch(packed, absmax, blocksize: int, code, shape, dtype, chunk_bytes: int = 1 << 23):
    """The reference's torch decode on the CPU (selas/codecs.py:155-199): a [256, 2] fp32 table maps a byte
    to (code[hi], code[lo]); rows of a blocksize-wide view are multiplied by their absmax in fp32 and
    copied (rounded once) into the output, 8 MiB of codes at a time. The same values as ``decode``; this
    is the path the benchmark times as the reference's CPU linear."""
    import torch

    packed = torch.as_tensor(packed).reshape(-1)
    absmax = torch.as_tensor(absmax).reshape(-1)
    n_bytes = packed.numel()
    out = torch.empty(n_bytes * 2, dtype=dtype)
    c = torch.tensor([float(v) for v in code], dtype=torch.float32)
    b = torch.arange(256)
    lut = torch.stack((c[b >> 4], c[b & 15]), dim=1)
    bpb = blocksize // 2
    step = max(bpb, (chunk_bytes // bpb) * bpb)
    for s in range(0, n_bytes, step):
        e = min(n_bytes, s + step)
        vals = lut.index_select(0, packed[s:e].to(torch.int32)).view(-1, blocksize)
        vals.mul_(absmax[s // bpb:e // bpb].unsqueeze(1))
        out[2 * s:2 * e].copy_(vals.view(-1))
    return out.view(tuple(shape))
