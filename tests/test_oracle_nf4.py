"""Pins the NF4 oracle (oracle/nf4.py, oracle/nf4_ref.c) independently of its own formulas.

Checks: the reference's known-answer packing test (selas tests/test_codecs.py:47-51),
the nearest-code invariant by brute force over all 16 codes (test_codecs.py:66-75),
exact decodes where the fp32 product is exact, the midpoint tie rule and NaN rule of
torch.bucketize, the relative-error bound (test_codecs.py:62-63), numpy vs C, and the
fp32 -> bf16 / fp16 roundings against torch's own casts.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4

CODE = np.asarray(nf4.NF4_CODE, dtype=np.float32)


def test_packing_known_answer_high_nibble_first():
    # selas tests/test_codecs.py:47-51: [-1, 1, 0 x 62] -> byte 0 = (0 << 4) | 15, absmax 1
    t = np.array([-1.0, 1.0] + [0.0] * 62, dtype=np.float32)
    for enc in (nf4.encode, nf4.c_encode):
        packed, absmax = enc(t)
        assert packed[0] == 0x0F and absmax[0] == 1.0
        assert (packed[1:] == 0x77).all()  # 0.0 is code 7 in both nibbles


def test_encode_picks_nearest_code_by_brute_force():
    rng = np.random.default_rng(2)
    t = rng.standard_normal(64 * 200).astype(np.float32)
    packed, absmax = nf4.encode(t)
    idx = np.empty(t.size, dtype=np.int64)
    idx[0::2], idx[1::2] = packed >> 4, packed & 15
    normed = (t.reshape(-1, 64) / absmax[:, None]).reshape(-1)
    dist = np.abs(normed[:, None] - CODE[None, :])
    best = dist.min(axis=1)
    assert np.allclose(dist[np.arange(t.size), idx], best, atol=1e-6)
    # ties excluded, the chosen code is the unique nearest one
    unique = (np.sort(dist, axis=1)[:, 1] - best) > 1e-6
    assert (idx[unique] == dist.argmin(axis=1)[unique]).all()


def test_ties_go_to_the_lower_code_and_nan_to_the_top():
    mids = nf4.midpoints()
    # a block whose absmax is 1 (the first element), then every midpoint exactly
    t = np.zeros(64, dtype=np.float32)
    t[0] = 1.0
    t[2:17] = mids
    packed, _ = nf4.encode(t)
    idx = np.empty(64, dtype=np.int64)
    idx[0::2], idx[1::2] = packed >> 4, packed & 15
    assert idx[0] == 15
    assert list(idx[2:17]) == list(range(15))  # x == mids[i] -> code i (the lower neighbour)
    # torch.bucketize itself (the reference's call) agrees on ties, +-inf and NaN
    x = np.array([np.nan, np.inf, -np.inf, *mids], dtype=np.float32)
    ref = torch.bucketize(torch.from_numpy(x), torch.from_numpy(mids)).numpy()
    ours = np.searchsorted(mids, x, side="left")
    assert (ref == ours).all() and ref[0] == 15


def test_decode_is_exact_with_power_of_two_scales():
    # every byte value, each block scaled by a distinct power of two: products are exact
    for bs in (2, 32, 64, 128):
        packed = np.arange(256, dtype=np.uint8).repeat(2)
        nblk = packed.size * 2 // bs
        absmax = (2.0 ** (np.arange(nblk) % 7 - 3)).astype(np.float32)
        out = nf4.decode(packed, absmax, bs)
        k = np.arange(out.size)
        nib = np.where(k % 2 == 0, packed[k // 2] >> 4, packed[k // 2] & 15)
        assert (out == CODE[nib] * absmax[k // bs]).all()


def test_reconstruction_error_bound_on_gaussians():
    rng = np.random.default_rng(1)
    t = rng.standard_normal(96 * 128).astype(np.float32)
    packed, absmax = nf4.encode(t)
    deq = nf4.decode(packed, absmax, 64)
    rel = np.linalg.norm(deq - t) / np.linalg.norm(t)
    assert rel < 0.12  # selas tests/test_codecs.py:62-63


def test_zero_block_and_nan_block():
    t = np.zeros(128, dtype=np.float32)
    t[64:] = 1.0
    t[70] = np.nan
    packed, absmax = nf4.encode(t)
    assert absmax[0] == 0.0 and (packed[:32] == 0x77).all()  # absmax 0 -> divide by 1 -> code of 0.0
    assert np.isnan(absmax[1])
    pc, ac = nf4.c_encode(t)
    assert (pc == packed).all() and ac[0] == 0.0 and np.isnan(ac[1])


@pytest.mark.parametrize("bs", [2, 64, 256])
def test_numpy_and_c_restatements_agree(bs):
    rng = np.random.default_rng(bs)
    t = (rng.standard_normal(bs * 97) * rng.choice([1e-30, 1e-3, 1.0, 3e4], size=bs * 97)).astype(np.float32)
    p1, a1 = nf4.encode(t, bs)
    p2, a2 = nf4.c_encode(t, bs)
    assert (p1 == p2).all() and (a1.view(np.uint32) == a2.view(np.uint32)).all()
    for out in (nf4.F32, nf4.F16, nf4.BF16):
        d1, d2 = nf4.decode(p1, a1, bs, out=out), nf4.c_decode(p1, a1, bs, out=out)
        assert (d1.view(np.uint8) == d2.view(np.uint8)).all()


def test_roundings_match_torch_casts():
    rng = np.random.default_rng(5)
    with np.errstate(over="ignore"):
        v = np.concatenate([rng.standard_normal(50_000).astype(np.float32) * s
                            for s in (1e-40, 1e-8, 6e-8, 1e-5, 1e-3, 1.0, 6.5e4, 7e4, 3e38)])
    # exact ties for bf16: low 16 bits = 0x8000
    ties = (rng.integers(0, 2**31, 1000, dtype=np.uint32) & 0xFFFF0000 | 0x8000).view(np.float32)
    ties = ties[np.isfinite(ties)]  # NaN payloads are not part of the contract
    v = np.concatenate([v, ties, np.array([np.inf, -np.inf, 0.0, -0.0], dtype=np.float32)])
    tv = torch.from_numpy(v)
    assert (nf4.bf16_bits(v) == tv.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)).all()
    with np.errstate(over="ignore"):
        assert (nf4.f16_bits(v) == tv.to(torch.float16).view(torch.int16).numpy().view(np.uint16)).all()
    lib = nf4.c_lib()
    sub = v[::37]
    c = np.array([lib.nf4o_f16_bits(float(x)) for x in sub], dtype=np.uint16)
    assert (c == torch.from_numpy(sub).to(torch.float16).view(torch.int16).numpy().view(np.uint16)).all()


def test_encode_rejects_partial_blocks():
    with pytest.raises(ValueError):
        nf4.encode(np.zeros(100, dtype=np.float32), 64)
    with pytest.raises(ValueError):
        nf4.encode(np.zeros(63, dtype=np.float32), 3)


def test_torch_restatement_equals_the_c_and_numpy_decodes():
    # The torch decode the benchmark times as the reference's CPU path gives the bits of the pinned decodes,
    # across chunk boundaries (chunk of 96 bytes over a 1000-byte tensor) and for every output type.
    import torch

    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, 1024, dtype=np.uint8)
    absmax = (rng.random(32, dtype=np.float32) * 3).astype(np.float32)
    absmax[3] = 0.0
    for dt, out in ((torch.float32, nf4.F32), (torch.float16, nf4.F16), (torch.bfloat16, nf4.BF16)):
        got = nf4.decode_torch(packed, absmax, 64, nf4.NF4_CODE, (2048,), dt, chunk_bytes=96)
        want = nf4.decode(packed, absmax, 64, out=out)
        bits = got.view(torch.int32 if dt == torch.float32 else torch.int16).numpy()
        assert (bits.view(np.uint32 if dt == torch.float32 else np.uint16) == want.view(bits.dtype).view(
            np.uint32 if dt == torch.float32 else np.uint16)).all()
