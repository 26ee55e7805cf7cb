"""NF4 weight codec with the reference's interface, on the gfx950 kernels.

Mirrors selas/codecs.py: the same names, argument order, return types and
errors (ValueError for bad sizes, NotImplementedError for a partial final
block), so that selas's store can call these in place of its own. Encoding and
decoding run on the GPU (libselas_amd.so); a tensor on the CPU is moved to the
current GPU for encoding (the reference encodes on the CPU at convert time and
returns CPU parts, which is kept), while decoding a CPU tensor is an error.

Format (selas/codecs.py:12-15, 99-119): blockwise absmax in fp32 over the
flattened tensor, two 4-bit codes per byte with the first element in the high
nibble, a 16-entry codebook in ``meta["code"]``.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import _lib

# The NormalFloat-4 codebook of QLoRA / bitsandbytes (selas/codecs.py:58-63). A
# format constant: NF4 checkpoints carry these exact fp32 values.
NF4_CODE: tuple[float, ...] = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)


class EncodedTensor(NamedTuple):
    """A tensor as codec parts, as selas/codecs.py:66-75."""

    name: str
    codec: str
    shape: tuple[int, ...]
    meta: dict
    parts: dict[str, torch.Tensor]

    @property
    def nbytes(self) -> int:
        return sum(p.numel() * p.element_size() for p in self.parts.values())


def encode_raw(name: str, t: torch.Tensor, dtype: torch.dtype | None = None) -> EncodedTensor:
    """Stores a tensor as-is (selas/codecs.py:80-83); no kernel involved."""
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return EncodedTensor(name, "raw", tuple(t.shape), {}, {"data": t.contiguous()})


def _gpu_for(t: torch.Tensor) -> torch.device:
    if t.device.type == "cuda":
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("selas_amd encodes on the GPU and none is available")
    return torch.device("cuda", torch.cuda.current_device())


def encode_nf4(name: str, t: torch.Tensor, blocksize: int = 64, code: tuple[float, ...] = NF4_CODE) -> EncodedTensor:
    """NF4-encodes ``t`` (selas/codecs.py:99-119) with the GPU encoder.

    Returns parts on the device ``t`` lives on: a CPU tensor is encoded on the
    current GPU and its parts are copied back, as the reference's convert step
    expects CPU parts.
    """
    n = t.numel()
    if blocksize <= 0 or n % blocksize or blocksize % 2:
        raise ValueError(f"nf4 needs numel divisible by blocksize ({n} % {blocksize}) for {name}")
    dev = _gpu_for(t)
    flat = t.detach().to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    packed = torch.empty(n // 2, dtype=torch.uint8, device=dev)
    absmax = torch.empty(n // blocksize, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("selas_nf4_encode", flat.data_ptr(), n, blocksize, _lib.code_array(code), packed.data_ptr(),
                  absmax.data_ptr(), _lib.stream(dev))
    if t.device.type != "cuda":
        packed, absmax = packed.cpu(), absmax.cpu()
    return EncodedTensor(name, "nf4", tuple(t.shape), {"blocksize": blocksize, "code": list(code)},
                         {"packed": packed, "absmax": absmax})


def nf4_import(
    name: str,
    packed: torch.Tensor,
    absmax: torch.Tensor,
    shape: tuple[int, ...],
    blocksize: int,
    code: list[float] | tuple[float, ...],
) -> EncodedTensor:
    """Wraps existing bnb NF4 bits without touching them (selas/codecs.py:122-145)."""
    n = 1
    for s in shape:
        n *= int(s)
    if n % blocksize:
        raise NotImplementedError(f"{name}: partial final NF4 block ({n} % {blocksize}) is not supported")
    packed = packed.reshape(-1).contiguous()
    if packed.dtype != torch.uint8 or packed.numel() * 2 != n:
        raise ValueError(f"{name}: packed NF4 data has {packed.numel()} bytes for {n} elements")
    absmax = absmax.reshape(-1).float().contiguous()
    if absmax.numel() != n // blocksize:
        raise ValueError(f"{name}: expected {n // blocksize} absmax values, got {absmax.numel()}")
    return EncodedTensor(
        name, "nf4", tuple(int(s) for s in shape), {"blocksize": int(blocksize), "code": [float(c) for c in code]},
        {"packed": packed, "absmax": absmax},
    )


def nf4_dequant(packed: torch.Tensor, absmax: torch.Tensor, blocksize: int, code, shape, dtype: torch.dtype) -> torch.Tensor:
    """Decodes to ``dtype``: code[nibble] * absmax[block] in fp32, rounded once.

    Bit-identical to the reference decode (selas/codecs.py:178-199, 260-266).
    """
    dev = _lib.require_gpu(packed, absmax)
    if packed.dtype != torch.uint8:
        raise ValueError(f"packed NF4 data must be uint8, got {packed.dtype}")
    if absmax.dtype != torch.float32:
        raise ValueError(f"NF4 absmax must be float32, got {absmax.dtype}")
    packed = packed.reshape(-1)
    absmax = absmax.reshape(-1)
    if not packed.is_contiguous() or not absmax.is_contiguous():
        raise ValueError("NF4 parts must be contiguous")
    n_bytes = packed.numel()
    bs = int(blocksize)
    if bs <= 0 or bs % 2 or (2 * n_bytes) % bs or absmax.numel() < (2 * n_bytes) // bs:
        raise ValueError(f"NF4 parts do not match: {n_bytes} bytes, {absmax.numel()} absmax, blocksize {bs}")
    out = torch.empty(n_bytes * 2, dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.call("selas_nf4_dequant", packed.data_ptr(), absmax.data_ptr(), n_bytes, bs, _lib.code_array(code),
                  out.data_ptr(), _lib.dtype_code(dtype), _lib.stream(dev))
    return out.view(tuple(shape))


def encode_int8_row(name: str, t: torch.Tensor) -> EncodedTensor:
    """int8_row-encodes ``t`` (selas/codecs.py:86-96) with the GPU encoder: one fp32 scale per row
    (absmax / 127, 1 for a zero row) and q = clamp(round(w / scale), -127, 127) in ``t``'s shape.

    Parts live on ``t``'s device; a CPU tensor is encoded on the current GPU and its parts are
    copied back, as for ``encode_nf4``.
    """
    if t.dim() < 2:
        raise ValueError(f"int8_row needs a matrix, got {tuple(t.shape)} for {name}")
    dev = _gpu_for(t)
    rows = int(t.shape[0])
    cols = t.numel() // rows if rows else 0
    w = t.detach().to(device=dev, dtype=torch.float32).reshape(rows, cols).contiguous()
    q = torch.empty(tuple(t.shape), dtype=torch.int8, device=dev)
    scale = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("selas_int8_row_encode", w.data_ptr(), rows, cols, q.data_ptr(), scale.data_ptr(), _lib.stream(dev))
    if t.device.type != "cuda":
        q, scale = q.cpu(), scale.cpu()
    return EncodedTensor(name, "int8_row", tuple(t.shape), {}, {"q": q, "scale": scale})


def int8_row_dequant(q: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Decodes to ``dtype`` in q's shape: ``q.to(dtype) * scale.to(dtype)`` per row, evaluated in ``dtype``.

    Bit-identical to the reference decode (selas/codecs.py:273-277).
    """
    dev = _lib.require_gpu(q, scale)
    if q.dtype != torch.int8:
        raise ValueError(f"int8_row data must be int8, got {q.dtype}")
    if scale.dtype != torch.float32:
        raise ValueError(f"int8_row scale must be float32, got {scale.dtype}")
    if q.dim() < 1 or scale.numel() != q.shape[0] or not q.is_contiguous() or not scale.is_contiguous():
        raise ValueError(f"int8_row parts do not match: q {tuple(q.shape)}, scale {tuple(scale.shape)} "
                         "(one scale per row, contiguous)")
    rows = int(q.shape[0])
    cols = q.numel() // rows if rows else 0
    out = torch.empty(tuple(q.shape), dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.call("selas_int8_row_dequant", q.data_ptr(), scale.data_ptr(), rows, cols, out.data_ptr(),
                  _lib.dtype_code(dtype), _lib.stream(dev))
    return out


def decode(codec: str, parts: dict[str, torch.Tensor], meta: dict, shape: tuple[int, ...], dtype: torch.dtype) -> torch.Tensor:
    """Codec dispatch as selas/codecs.py:269-280 (raw, int8_row and nf4)."""
    if codec == "raw":
        x = parts["data"]
        return x if x.dtype == dtype else x.to(dtype)
    if codec == "nf4":
        return nf4_dequant(parts["packed"], parts["absmax"], int(meta["blocksize"]), meta["code"], tuple(shape), dtype)
    if codec == "int8_row":
        return int8_row_dequant(parts["q"], parts["scale"], dtype)
    raise ValueError(f"unknown codec {codec!r}")


def decoded_is_view(codec: str, stored_dtype: str | None, dtype: torch.dtype) -> bool:
    """True when decoding is a zero-copy view (selas/codecs.py:283-284)."""
    return codec == "raw" and stored_dtype is not None and str(dtype).removeprefix("torch.") == stored_dtype
