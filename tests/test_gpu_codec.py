"""NF4 decode/encode on the GPU, bit-exact against the oracle (oracle/nf4.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4 as onf4
from selas_amd import codecs

from .conftest import seeded

pytestmark = pytest.mark.gpu

OUT = {torch.float32: onf4.F32, torch.float16: onf4.F16, torch.bfloat16: onf4.BF16}


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def oracle_bits(packed, absmax, bs, dt):
    r = onf4.decode(packed.cpu().numpy(), absmax.cpu().numpy(), bs, out=OUT[dt])
    return r.view(np.uint32) if dt == torch.float32 else r


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_reference_self_check_vectors(dev, dt):
    # the recipe of the reference's runtime self-check (selas/codecs.py:244-252)
    g = seeded(0)
    packed = torch.randint(0, 256, (4096,), dtype=torch.uint8, generator=g)
    absmax = torch.rand(128, generator=g) + 0.01
    out = codecs.nf4_dequant(packed.to(dev), absmax.to(dev), 64, codecs.NF4_CODE, (8192,), dt)
    assert (bits(out) == oracle_bits(packed, absmax, 64, dt)).all()


@pytest.mark.parametrize("bs", [2, 6, 32, 64, 128, 4096])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_decode_bit_exact_any_blocksize(dev, bs, dt):
    g = seeded(bs)
    n_bytes = bs * 37 // 2 if bs > 2 else 1001
    packed = torch.randint(0, 256, (n_bytes,), dtype=torch.uint8, generator=g)
    nblk = 2 * n_bytes // bs
    absmax = torch.randn(nblk, generator=g).abs() * torch.tensor([1e-30, 1e-6, 1.0, 3e4, 1e38])[torch.arange(nblk) % 5]
    absmax[::7] = 0.0
    out = codecs.nf4_dequant(packed.to(dev), absmax.to(dev), bs, codecs.NF4_CODE, (2 * n_bytes,), dt)
    assert (bits(out) == oracle_bits(packed, absmax, bs, dt)).all()


def test_decode_unaligned_views_and_tails(dev):
    g = seeded(3)
    buf = torch.randint(0, 256, (4096 + 64,), dtype=torch.uint8, generator=g).to(dev)
    absmax = (torch.rand(200, generator=g) + 0.5).to(dev)
    for off, nb in [(1, 2048), (3, 1008), (32, 2080), (0, 16), (5, 48)]:  # whole blocks of 16 bytes
        p = buf[off: off + nb]
        out = codecs.nf4_dequant(p, absmax, 32, codecs.NF4_CODE, (2 * nb,), torch.bfloat16)
        assert (bits(out) == oracle_bits(p, absmax, 32, torch.bfloat16)).all(), (off, nb)


def test_decode_with_a_custom_codebook(dev):
    code = tuple(float(c) for c in np.linspace(-2, 1.5, 16, dtype=np.float32) ** 3)
    g = seeded(4)
    packed = torch.randint(0, 256, (512,), dtype=torch.uint8, generator=g)
    absmax = torch.rand(16, generator=g) + 0.1
    out = codecs.nf4_dequant(packed.to(dev), absmax.to(dev), 64, code, (1024,), torch.float32)
    ref = onf4.decode(packed.numpy(), absmax.numpy(), 64, code, onf4.F32)
    assert (bits(out) == ref.view(np.uint32)).all()


@pytest.mark.parametrize("bs", [64, 32, 256])
def test_encode_byte_exact(dev, bs):
    g = seeded(10 + bs)
    w = torch.randn(96, 4 * bs, generator=g) * 0.02
    w[3] = 0.0
    w[5, :bs] = torch.linspace(-1, 1, bs)
    e = codecs.encode_nf4("w", w.to(dev), bs)
    p_ref, a_ref = onf4.encode(w.numpy(), bs)
    assert e.parts["packed"].device.type == "cuda"
    assert (e.parts["packed"].cpu().numpy() == p_ref).all()
    assert (e.parts["absmax"].cpu().numpy().view(np.uint32) == a_ref.view(np.uint32)).all()
    assert e.meta == {"blocksize": bs, "code": list(codecs.NF4_CODE)} and e.shape == (96, 4 * bs)


def test_encode_ties_and_specials(dev):
    mids = onf4.midpoints()
    t = np.zeros(128, dtype=np.float32)
    t[0] = 1.0
    t[2:17] = mids
    t[64:] = np.float32(2.5) * np.linspace(-1, 1, 64, dtype=np.float32)
    e = codecs.encode_nf4("w", torch.from_numpy(t).to(dev), 64)
    p_ref, a_ref = onf4.encode(t, 64)
    assert (e.parts["packed"].cpu().numpy() == p_ref).all() and (e.parts["absmax"].cpu().numpy() == a_ref).all()


def test_cpu_input_gives_cpu_parts_like_the_reference():
    w = torch.randn(8, 64, generator=seeded(5))
    e = codecs.encode_nf4("w", w)
    assert e.parts["packed"].device.type == "cpu"
    p_ref, _ = onf4.encode(w.numpy())
    assert (e.parts["packed"].numpy() == p_ref).all()


def test_round_trip_at_full_linear_size(dev):
    # config-1 weight 12288 x 3072, N(0, 0.02), seed 0: encode on the GPU, decode on the GPU,
    # both byte/bit-exact against the oracle, plus the reconstruction bound
    g = seeded(0)
    w = torch.randn(12288, 3072, generator=g) * 0.02
    e = codecs.encode_nf4("w", w.to(dev))
    p_ref, a_ref = onf4.c_encode(w.numpy()) if onf4.c_lib() else onf4.encode(w.numpy())
    assert (e.parts["packed"].cpu().numpy() == p_ref).all()
    assert (e.parts["absmax"].cpu().numpy() == a_ref).all()
    out = codecs.decode("nf4", e.parts, e.meta, e.shape, torch.bfloat16)
    assert out.shape == (12288, 3072)
    assert (bits(out).reshape(-1) == onf4.decode(p_ref, a_ref, 64, out=onf4.BF16)).all()
    rel = (out.float().cpu() - w).norm() / w.norm()
    assert rel < 0.12
