"""Fused attention (selas_amd.attention) on the GPU against an fp64 CPU reference of
softmax(q k^T / sqrt(Dh)) v, laid out as the reference's
SDPA(...).transpose(1, 2).reshape(B, L, H * Dh) (selas/models/flux.py:135-138).

Tolerance (the path's contract for floating-point kernels): max |y - ref| <= 1e-2 * max |ref|
and relative L2 <= 4e-3. The kernel rounds the probabilities to bf16 for the second product,
as torch's flash backends do; its output is bf16.
"""

from __future__ import annotations

import pytest
import torch

from selas_amd import _lib
from selas_amd import flux as F
from selas_amd.attention import attention, transpose_heads

from .conftest import seeded

pytestmark = pytest.mark.gpu

MAX_REL, L2_REL = 1e-2, 4e-3


def reference(q, k, v):
    """fp64 on the CPU: [B, H, L, Dh] -> [B, L, H * Dh]."""
    q, k, v = (t.double().cpu() for t in (q, k, v))
    b, h, l, d = q.shape
    s = q @ k.transpose(-1, -2) / d ** 0.5
    o = torch.softmax(s, dim=-1) @ v
    return o.transpose(1, 2).reshape(b, l, h * d)


def check_close(y, ref):
    y = y.double().cpu()
    err = (y - ref).abs().max().item()
    assert err <= MAX_REL * ref.abs().max().item(), f"max abs err {err} vs max {ref.abs().max().item()}"
    rel = ((y - ref).norm() / ref.norm()).item()
    assert rel <= L2_REL, f"relative L2 {rel}"


def qkv(b, h, l, seed, q_scale=1.0, dev="cuda"):
    g = seeded(seed)
    q = (torch.randn(b, h, l, 128, generator=g) * q_scale).to(torch.bfloat16)
    k = torch.randn(b, h, l, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(b, h, l, 128, generator=g).to(torch.bfloat16)
    return q.to(dev), k.to(dev), v.to(dev)


@pytest.mark.parametrize("b,h,l", [(1, 2, 128), (2, 3, 256), (1, 2, 640), (1, 1, 1536)])
def test_attention_matches_reference(dev, b, h, l):
    q, k, v = qkv(b, h, l, b + h + l)
    y = attention(q, k, v)
    assert y.shape == (b, l, h * 128) and y.dtype == torch.bfloat16
    check_close(y, reference(q, k, v))


@pytest.mark.parametrize("q_scale", [4.0, 12.0])
def test_attention_sharp_scores(dev, q_scale):
    # Scores spread over tens of units: the running maximum moves by more than the rescale
    # threshold many times, and most probabilities underflow.
    q, k, v = qkv(1, 2, 512, 7, q_scale)
    check_close(attention(q, k, v), reference(q, k, v))


def test_attention_maximum_in_the_last_tile(dev):
    # Each query's largest score sits in the last key tile: every earlier tile is rescaled away.
    q, k, v = qkv(1, 2, 384, 8)
    k = k.clone()
    k[:, :, -5:] = (q[:, :, :5].float() * 3).to(torch.bfloat16)
    check_close(attention(q, k, v), reference(q, k, v))


def test_attention_full_size_sample(dev):
    # One FLUX 1024^2 block: B = 1, H = 24, L = 4608 (512 text + 4096 image tokens); 2 heads x 96
    # sampled queries checked against the reference.
    q, k, v = qkv(1, 24, 4608, 9)
    y = attention(q, k, v).view(1, 4608, 24, 128)
    g = seeded(10)
    for hh in (0, 17):
        rows = torch.randint(0, 4608, (96,), generator=g)
        ref = reference(q[:, hh:hh + 1, rows], k[:, hh:hh + 1], v[:, hh:hh + 1]).view(1, 96, 128)
        check_close(y[:, rows, hh], ref)
    assert torch.isfinite(y).all()


def test_attention_deterministic_and_matches_sdpa(dev):
    q, k, v = qkv(2, 4, 1024, 11)
    y1, y2 = attention(q, k, v), attention(q, k, v)
    assert torch.equal(y1, y2)
    check_close(y1, reference(q, k, v))
    check_close(F.sdpa_attention(q, k, v), reference(q, k, v))  # the library path meets the same bound


@pytest.mark.parametrize("l", [256, 100, 1])
def test_transpose_heads_exact(dev, l):
    # [B, H, Dh, Lp], Lp = L rounded up to 64, the columns past L zero.
    v = torch.randn(3, 2, l, 128, generator=seeded(12)).to(torch.bfloat16).to(dev)
    vt = transpose_heads(v)
    lp = (l + 63) // 64 * 64
    assert vt.shape == (3, 2, 128, lp)
    assert torch.equal(vt[..., :l], v.transpose(-1, -2)) and torch.count_nonzero(vt[..., l:]) == 0


@pytest.mark.parametrize("b,h,l", [(1, 2, 1), (2, 2, 65), (1, 3, 100), (1, 2, 130), (2, 1, 1000), (1, 2, 3100)])
def test_any_sequence_length(dev, b, h, l):
    # L not a multiple of the 64-key tile or of the query tile (3100: eight waves per workgroup):
    # the last key tile is masked, the last query tile stored in part. FLUX at other resolutions
    # (e.g. 768 x 1360: 4080 image + 512 text tokens) has such lengths.
    q, k, v = qkv(b, h, l, 40 + l)
    y = attention(q, k, v)
    assert y.shape == (b, l, h * 128)
    check_close(y, reference(q, k, v))
    wide = torch.full((b * l + 3, h * 128 + 8), 7.0, dtype=torch.bfloat16, device=dev)
    out = wide[:b * l].view(b, l, h * 128 + 8)[..., :h * 128]
    attention(q, k, v, out=out)
    assert torch.equal(out, y)
    assert (wide[b * l:] == 7.0).all() and (wide[:, h * 128:] == 7.0).all()  # nothing written past the output


def test_unsupported_shapes_fall_back_to_sdpa(dev):
    l, d = 256, 64
    g = seeded(l + d)
    q, k, v = (torch.randn(1, 2, l, d, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    with pytest.raises(_lib.Unsupported):
        attention(q, k, v)
    y = F.attention(q, k, v)
    assert y.shape == (1, l, 2 * d)
    check_close(y, reference(q, k, v))


def test_attention_into_strided_rows(dev):
    # Output written into the first H*Dh columns of a wider buffer (linear2's input in the single block).
    q, k, v = qkv(2, 3, 256, 13)
    wide = torch.zeros(2, 256, 3 * 128 + 200, dtype=torch.bfloat16, device=dev)
    y = attention(q, k, v, out=wide[..., :3 * 128])
    assert y.data_ptr() == wide.data_ptr()
    assert torch.equal(wide[..., :3 * 128], attention(q, k, v))
    assert torch.count_nonzero(wide[..., 3 * 128:]) == 0


@pytest.mark.parametrize("b,h,l", [(2, 2, 3072), (1, 3, 3328)])
def test_eight_wave_workgroups(dev, b, h, l):
    # L >= 3072 runs 256 queries per workgroup (8 waves); the result meets the same bound, and a
    # strided destination gets the same bits.
    q, k, v = qkv(b, h, l, l + h)
    y = attention(q, k, v)
    g = seeded(l)
    rows = torch.randint(0, l, (128,), generator=g)
    for hh in range(h):
        ref = reference(q[:, hh:hh + 1, rows], k[:, hh:hh + 1], v[:, hh:hh + 1]).view(b, 128, 128)
        check_close(y.view(b, l, h, 128)[:, rows, hh], ref)
    wide = torch.zeros(b, l, h * 128 + 64, dtype=torch.bfloat16, device=dev)
    attention(q, k, v, out=wide[..., :h * 128])
    assert torch.equal(wide[..., :h * 128], y) and torch.count_nonzero(wide[..., h * 128:]) == 0
