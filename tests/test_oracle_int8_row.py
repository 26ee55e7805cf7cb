"""The int8_row oracle (oracle/int8_row.py) pinned against the reference's own test and
closed forms that a plausible mistake (wrong divisor, truncation instead of rounding, a
missing clamp, the scale unrounded in decode) would fail."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import int8_row as I
from oracle import nf4 as N

from .conftest import seeded


def test_reference_error_bound_with_outlier_row():
    # selas tests/test_codecs.py:37-45: seed 0, randn(64, 256), row 3 scaled by 50, fp32 decode,
    # per-row relative error < 0.01.
    t = torch.randn(64, 256, generator=torch.Generator().manual_seed(0))
    t[3] *= 50
    q, s = I.encode(t.numpy())
    out = I.decode(q, s, I.F32)
    rel = np.linalg.norm(out - t.numpy(), axis=1) / np.linalg.norm(t.numpy(), axis=1)
    assert rel.max() < 0.01


def test_multiples_of_the_scale_round_trip_exactly():
    # A row whose max is 127 has scale 1: integer entries are their own codes.
    row = np.arange(-127, 128, dtype=np.float32)
    w = np.stack([row, row * 0.5, row * 4.0])
    q, s = I.encode(w)
    assert s.tolist() == [1.0, 0.5, 4.0]
    assert np.array_equal(q[0], row.astype(np.int8)) and np.array_equal(q[1], q[0]) and np.array_equal(q[2], q[0])
    assert np.array_equal(I.decode(q, s, I.F32), w)


def test_ties_round_to_even_and_zero_rows():
    w = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5], [0.0] * 8], dtype=np.float32)
    q, s = I.encode(w)
    assert s.tolist() == [1.0, 1.0]
    assert q[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 4] and q[1].tolist() == [0] * 8


def test_every_code_is_the_nearest_level():
    # Brute force over all 255 levels of each row.
    w = (torch.randn(16, 96, generator=seeded(5)) * torch.rand(16, 1, generator=seeded(6)) * 10).numpy()
    q, s = I.encode(w)
    levels = np.arange(-127, 128, dtype=np.float64)
    for r in range(w.shape[0]):
        x = w[r].astype(np.float64) / np.float64(s[r])
        best = np.abs(x[:, None] - levels[None, :]).min(axis=1)
        assert np.all(np.abs(x - q[r]) <= best + 1e-4)
    assert np.abs(q).max() == 127 and s.dtype == np.float32


def test_shape_is_kept_and_vectors_rejected():
    w = np.ones((4, 3, 8), np.float32)
    q, s = I.encode(w)
    assert q.shape == (4, 3, 8) and s.shape == (4,)
    with pytest.raises(ValueError):
        I.encode(np.ones(8, np.float32))


@pytest.mark.parametrize("out,dt", [(I.BF16, torch.bfloat16), (I.F16, torch.float16), (I.F32, torch.float32)])
def test_decode_roundings_match_torch(out, dt):
    # The reference evaluates q.to(dt) * scale.to(dt) in dt; torch on the CPU gives those bits.
    g = seeded(7)
    q = torch.randint(-127, 128, (40, 64), generator=g, dtype=torch.int8)
    s = (torch.rand(40, generator=g) * 0.05 + 1e-4).float()
    ref = q.to(dt) * s.to(dt).view(-1, 1)
    got = I.decode(q.numpy(), s.numpy(), out)
    if out == I.F32:
        assert np.array_equal(got, ref.numpy())
    else:
        assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))


def test_decode_rounds_the_scale_first():
    # bf16: the scale is rounded before the product. 1 + 3 * 2^-10 rounds to 1, so q = 127 decodes to
    # exactly 127; the unrounded scale would give 127.37, which rounds to 127.5.
    s = np.array([1.0 + 3 * 2.0 ** -10], np.float32)
    q = np.array([[127]], np.int8)
    assert N.bf16_to_f32(I.decode(q, s, I.BF16))[0, 0] == 127.0
