"""int8_row codec oracle (numpy): test infrastructure only.

Restates selas/codecs.py:
  * ``encode`` — encode_int8_row (codecs.py:86-96): the weight as [rows, -1]
    in fp32, absmax per row, scale = absmax / 127 in fp32 (1 where absmax is not
    > 0), q = clamp(round_half_even(w / scale), -127, 127) as int8.
  * ``decode`` — the int8_row branch of decode (codecs.py:273-277):
    ``q.to(dt) * scale.to(dt)`` evaluated in dt: q converts exactly, the scale
    is rounded to dt, the product is formed in fp32 (exact for bf16 and fp16
    operands) and rounded once to dt.

Pinned by (tests/test_oracle_int8_row.py): the reference's own error-bound test
with its outlier row (test_codecs.py:37-45), closed forms (rows that are
multiples of their scale decode exactly; the round-half-even tie rule; the
zero row's scale of 1; the clamp), the nearest-level invariant by brute force
over all 255 levels, and the decode roundings against torch's own
``q.to(dt) * s.to(dt)``.
"""

from __future__ import annotations

import numpy as np

from .nf4 import BF16, F16, F32, bf16_to_f32, round_to  # noqa: F401  (dtype codes shared with the NF4 oracle)


def encode(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(q int8 in w's shape, scale fp32 [rows]) for a weight with at least 2 dimensions."""
    w = np.asarray(w, dtype=np.float32)
    if w.ndim < 2:
        raise ValueError(f"int8_row needs a matrix, got {w.shape}")
    rows = w.reshape(w.shape[0], -1)
    with np.errstate(invalid="ignore", divide="ignore"):
        absmax = np.abs(rows).max(axis=1).astype(np.float32) if rows.shape[1] else np.zeros(rows.shape[0], np.float32)
        scale = np.where(absmax > 0, absmax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
        v = np.rint(rows / scale[:, None]).astype(np.float32)
    q = np.clip(v, -127, 127).astype(np.int8)
    return q.reshape(w.shape), scale


def scale_as(scale: np.ndarray, out: int) -> np.ndarray:
    """The row scales rounded to the output type (as fp32 values)."""
    s = np.asarray(scale, dtype=np.float32)
    if out == F32:
        return s
    if out == F16:
        return s.astype(np.float16).astype(np.float32)
    return bf16_to_f32(round_to(s, BF16))


def decode(q: np.ndarray, scale: np.ndarray, out: int = F32) -> np.ndarray:
    """Reference int8_row decode: fp32 values (out=F32) or fp16/bf16 bit patterns, in q's shape."""
    q = np.asarray(q, dtype=np.int8)
    rows = q.reshape(q.shape[0], -1).astype(np.float32)
    vals = rows * scale_as(scale, out)[:, None]
    return round_to(vals.astype(np.float32), out).reshape(q.shape)
