"""The quantized-linear forward, with the reference's ``UnitView`` interface.

The reference decodes an NF4 weight to a bf16 temporary and calls ``F.linear``
(selas/store.py:289-293, codecs.py:269-280). ``nf4_linear`` computes the same
``x @ W.T + b`` with the decode fused into the GEMM operand load, so the
decoded weight never reaches memory. Shapes outside the fused kernels
(blocksize other than 64, K not a multiple of 64, dtypes other than bf16,
misaligned rows) keep the reference's convention: the weight is decoded (on the
GPU, by the bit-exact decode kernel) and a library GEMM runs.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from .codecs import EncodedTensor, decode, nf4_dequant


def _rows(x: torch.Tensor) -> torch.Tensor:
    """x as a 2-D [rows, K] view with unit column stride (copied only if no such view exists)."""
    k = x.shape[-1]
    if x.dim() == 2 and x.stride(-1) == 1:
        return x
    try:
        v = x.view(-1, k)
        if v.stride(-1) == 1:
            return v
    except RuntimeError:
        pass
    return x.reshape(-1, k).contiguous()


def nf4_linear(x: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor, blocksize: int, code, shape,
               bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, decode(W), bias)`` for an NF4 weight ``W`` of ``shape`` [N, K]."""
    n, k = int(shape[0]), int(shape[1])
    if len(shape) != 2:
        raise ValueError(f"linear weight must be 2-D, got {tuple(shape)}")
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects {k}")
    dev = _lib.require_gpu(x, packed, absmax, bias)
    x2 = _rows(x)
    m = x2.shape[0]
    y = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
    if bias is not None and (bias.dtype != x.dtype or not bias.is_contiguous()):
        bias = bias.to(x.dtype).contiguous()
    try:
        if x.dtype not in _lib.DTYPE_CODES:
            raise _lib.Unsupported(f"dtype {x.dtype}")
        with torch.cuda.device(dev):
            _lib.call("selas_nf4_linear", x2.data_ptr(), m, k, x2.stride(0), packed.data_ptr(), absmax.data_ptr(),
                      int(blocksize), _lib.code_array(code), n, _lib.ptr(bias), y.data_ptr(), n,
                      _lib.dtype_code(x.dtype), _lib.stream(dev))
        return y
    except _lib.Unsupported:
        w = nf4_dequant(packed, absmax, blocksize, code, (n, k), x.dtype)
        return F.linear(x, w, bias)


class UnitView:
    """Typed access to one unit's tensors, as selas.store.UnitView (store.py:242-293).

    ``tensors`` maps tensor names to :class:`EncodedTensor` whose parts live on
    the GPU. ``get`` decodes (raw tensors in the compute dtype are returned as
    zero-copy views and cached), ``linear`` is the quantized-linear forward.
    """

    __slots__ = ("tensors", "dtype", "_views")

    def __init__(self, tensors: dict[str, EncodedTensor], dtype: torch.dtype):
        self.tensors = tensors
        self.dtype = dtype
        self._views: dict[tuple, torch.Tensor] = {}

    def has(self, name: str) -> bool:
        return name in self.tensors

    def codec(self, name: str) -> str:
        return self.tensors[name].codec

    def parts(self, name: str) -> dict[str, torch.Tensor]:
        return self.tensors[name].parts

    def get(self, name: str, dtype: torch.dtype | None = None) -> torch.Tensor:
        dtype = dtype or self.dtype
        key = (name, dtype)
        hit = self._views.get(key)
        if hit is not None:
            return hit
        e = self.tensors[name]
        out = decode(e.codec, e.parts, e.meta, e.shape, dtype)
        if e.codec == "raw" and out.data_ptr() == e.parts["data"].data_ptr():
            self._views[key] = out
        return out

    def linear(self, x: torch.Tensor, prefix: str, dtype: torch.dtype | None = None) -> torch.Tensor:
        dtype = dtype or self.dtype
        e = self.tensors[prefix + ".weight"]
        bname = prefix + ".bias"
        b = self.get(bname, dtype) if bname in self.tensors else None
        if e.codec == "nf4" and x.dtype == dtype:
            return nf4_linear(x, e.parts["packed"], e.parts["absmax"], int(e.meta["blocksize"]), e.meta["code"],
                              e.shape, b)
        return F.linear(x, self.get(prefix + ".weight", dtype), b)
