"""The block attention of FLUX (selas/models/flux.py:135-138) as a gfx950 kernel.

The reference calls ``F.scaled_dot_product_attention(q, k, v)`` on q, k, v
[B, H, L, Dh] and returns ``out.transpose(1, 2).reshape(B, L, H * Dh)``.
``attention`` computes the same with one fused kernel that writes the
[B, L, H * Dh] layout directly (the transpose copy disappears). The values are
read transposed ([B, H, Dh, L] padded to a multiple of 64 tokens), produced by
``transpose_heads``. Any sequence length runs; shapes outside the kernel (head
dim other than 128, dtypes other than bf16) raise ``Unsupported``;
``flux.attention`` then runs SDPA, as the reference.
"""

from __future__ import annotations

import torch

from . import _lib


def _heads(t: torch.Tensor, what: str) -> torch.Tensor:
    if t.dim() != 4:
        raise ValueError(f"{what}: expected [B, H, L, Dh], got shape {tuple(t.shape)}")
    return t if t.is_contiguous() else t.contiguous()


def transpose_heads(v: torch.Tensor) -> torch.Tensor:
    """v [B, H, L, Dh] -> [B, H, Dh, Lp] (contiguous), Lp = L rounded up to 64 tokens; the
    columns past L are zero."""
    v = _heads(v, "transpose_heads")
    b, h, l, d = v.shape
    dev = _lib.require_gpu(v)
    if v.dtype not in _lib.DTYPE_CODES:
        raise _lib.Unsupported(f"transpose_heads: dtype {v.dtype}")
    vt = torch.empty(b, h, d, (l + 63) // 64 * 64, dtype=v.dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.call("selas_transpose_heads", v.data_ptr(), b * h, l, d, vt.data_ptr(), _lib.dtype_code(v.dtype),
                  _lib.stream(dev))
    return vt


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(q k^T / sqrt(Dh)) v over [B, H, L, Dh] -> [B, L, H * Dh].

    ``out``: optional [B, L, H * Dh] destination whose rows may be strided (e.g. the first
    H * Dh columns of a wider buffer); it is returned."""
    q, k = _heads(q, "attention"), _heads(k, "attention")
    if q.shape != k.shape or q.shape != v.shape or q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(f"attention: q {tuple(q.shape)} {q.dtype}, k {tuple(k.shape)} {k.dtype}, "
                         f"v {tuple(v.shape)} {v.dtype} must match")
    b, h, l, d = q.shape
    dev = _lib.require_gpu(q, k, v)
    if q.dtype not in _lib.DTYPE_CODES:
        raise _lib.Unsupported(f"attention: dtype {q.dtype}")
    if d != 128 or q.dtype != torch.bfloat16:
        raise _lib.Unsupported(f"attention: fused kernel takes bf16 and head_dim 128 (got {q.dtype}, {d})")
    if out is None:
        out = torch.empty(b, l, h * d, dtype=q.dtype, device=dev)
    elif (out.shape != (b, l, h * d) or out.dtype != q.dtype or out.device != q.device or out.stride(-1) != 1
          or out.stride(0) != l * out.stride(1)):
        raise ValueError(f"attention: out must be [{b}, {l}, {h * d}] {q.dtype} on {q.device} with unit column "
                         f"stride and equally spaced rows, got {tuple(out.shape)} strides {out.stride()}")
    vt = transpose_heads(v)
    with torch.cuda.device(dev):
        _lib.call("selas_attention", q.data_ptr(), k.data_ptr(), vt.data_ptr(), b, h, l, d, out.data_ptr(),
                  out.stride(1), _lib.dtype_code(q.dtype), _lib.stream(dev))
    return out
