"""The seven segment kernels against the oracle segments (oracle/segments.py), tiny and FLUX shapes.

Tolerance: outputs rounded to bf16 are compared with the oracle's fp32 values with
max |err| <= 1e-2 * max |ref| and relative L2 <= 4e-3; fp32 outputs (the residual
stream) to 1e-5 relative.
"""

from __future__ import annotations

import pytest
import torch

from oracle import segments as S
from selas_amd.kernels import Kernels

from .conftest import seeded

pytestmark = pytest.mark.gpu
K = Kernels()
BF = torch.bfloat16


def close(out, ref, max_rel=1e-2, l2=4e-3):
    out, ref = out.double().cpu(), ref.double().cpu()
    assert out.shape == ref.shape
    assert (out - ref).abs().max() <= max_rel * ref.abs().max()
    assert (out - ref).norm() <= l2 * ref.norm()


def mods(b, d, n, seed):
    m = torch.randn(b, n * d, generator=seeded(seed)) * 0.1
    return m, m.float().unsqueeze(1).chunk(n, dim=-1)


@pytest.mark.parametrize("b,l,d", [(1, 5, 64), (2, 33, 3072), (1, 4608, 3072), (3, 7, 1000)])
def test_mod_in(dev, b, l, d):
    x = torch.randn(b, l, d, generator=seeded(1)) * 2 + 0.5
    _, (sh, sc, _) = mods(b, d, 3, 2)
    out = K.mod_in(x.to(dev), sh.to(dev), sc.to(dev), BF)
    assert out.dtype == BF and out.shape == (b, l, d)
    close(out, S.mod_in(x, sh, sc, torch.float32))


def test_mod_in_strided_rows_and_fp32_output(dev):
    big = torch.randn(2, 40, 256, generator=seeded(3))
    x = big[:, 8:]  # final_layer's img = x[:, lt:] view
    _, (sh, sc) = mods(2, 256, 2, 4)
    out = K.mod_in(x.to(dev)[:, :], sh.to(dev), sc.to(dev), torch.float32)
    ref = S.mod_in(x, sh, sc, torch.float32)
    assert torch.allclose(out.cpu(), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("b,l,d", [(1, 4608, 3072), (2, 9, 64)])
@pytest.mark.parametrize("guard", [False, True])
def test_gated_add_and_gated_add_mod(dev, b, l, d, guard):
    x = torch.randn(b, l, d, generator=seeded(5))
    y = (torch.randn(b, l, d, generator=seeded(6)) * (1e5 if guard else 1)).to(torch.float16 if guard else BF)
    _, (sh, sc, g) = mods(b, d, 3, 7)
    out = K.gated_add(x.to(dev), g.to(dev), y.to(dev), guard)
    ref = S.gated_add(x, g, y, guard)
    assert out.dtype == torch.float32
    assert torch.allclose(out.cpu(), ref, rtol=1e-5, atol=1e-5 * ref.abs().max().item())
    xo, h = K.gated_add_mod(x.to(dev), g.to(dev), y.to(dev), sh.to(dev), sc.to(dev), BF, guard)
    xr, hr = S.gated_add(x, g, y, guard), S.mod_in(S.gated_add(x, g, y, guard), sh, sc, torch.float32)
    assert torch.allclose(xo.cpu(), xr, rtol=1e-5, atol=1e-5 * xr.abs().max().item())
    close(h, hr)


def rope(l, dh, seed):
    ang = torch.rand(l, dh // 2, generator=seeded(seed), dtype=torch.float64) * 40
    return ang.cos().float(), ang.sin().float()


@pytest.mark.parametrize("b,l,h,dh", [(1, 4608, 24, 128), (2, 17, 4, 16), (1, 3, 2, 128)])
def test_qkv_single(dev, b, l, h, dh):
    d = h * dh
    lin1 = torch.randn(b, l, 3 * d + 4 * d, generator=seeded(8)).to(BF)
    qkv = lin1[..., :3 * d]  # strided view of linear1's output, as in single_block
    qs = 1 + 0.02 * torch.randn(dh, generator=seeded(9))
    ks = 1 + 0.02 * torch.randn(dh, generator=seeded(10))
    cos, sin = rope(l, dh, 11)
    q, k, v = K.qkv_single(lin1.to(dev)[..., :3 * d], qs.to(dev), ks.to(dev), cos.to(dev), sin.to(dev), h, BF)
    qr, kr, vr = S.qkv_single(qkv, qs, ks, cos, sin, h, torch.float32)
    close(q, qr)
    close(k, kr)
    assert torch.equal(v.cpu(), vr) and v.is_contiguous() and q.shape == (b, h, l, dh)


@pytest.mark.parametrize("b,lt,li,h,dh", [(1, 512, 4096, 24, 128), (2, 5, 11, 4, 16)])
def test_qkv_double(dev, b, lt, li, h, dh):
    d = h * dh
    t = torch.randn(b, lt, 3 * d, generator=seeded(12)).to(BF)
    i = torch.randn(b, li, 3 * d, generator=seeded(13)).to(BF)
    sc = [1 + 0.02 * torch.randn(dh, generator=seeded(14 + j)) for j in range(4)]
    cos, sin = rope(lt + li, dh, 18)
    q, k, v = K.qkv_double(t.to(dev), i.to(dev), *(s.to(dev) for s in sc), cos.to(dev), sin.to(dev), h, BF)
    qr, kr, vr = S.qkv_double(t, i, *sc, cos, sin, h, torch.float32)
    close(q, qr)
    close(k, kr)
    assert torch.equal(v.cpu(), vr)


def test_gelu_and_attn_mlp(dev):
    h = torch.randn(1, 4608, 21504, generator=seeded(19)).to(BF)
    mlp = h[..., 9216:]
    attn = torch.randn(1, 4608, 3072, generator=seeded(20)).to(BF)
    out = K.attn_mlp(attn.to(dev), h.to(dev)[..., 9216:])
    ref = torch.cat((attn.float(), S.gelu(mlp.float())), dim=2)
    assert out.shape == (1, 4608, 15360)
    assert torch.equal(out[..., :3072].cpu(), attn)
    close(out[..., 3072:], ref[..., 3072:])
    g = K.gelu(h.to(dev)[..., :1000])
    close(g, S.gelu(h[..., :1000].float()))
    small = torch.randn(3, 7, generator=seeded(21)).to(BF)  # odd width: the scalar path
    close(K.gelu(small.to(dev)), S.gelu(small.float()))


def test_unsupported_calls_fall_back_to_the_eager_segment(dev):
    # Calls the kernels do not take run the eager segment on the GPU, with one warning per segment (as
    # selas's compiled segments fall back to eager ones, flux.py:215-235): a width that is not a multiple
    # of 4 (D = 1002), qkv rows 2 bytes off alignment, fp32 attn_mlp, a bf16 residual stream.
    import warnings

    from selas_amd import kernels

    kernels._warned.clear()
    b, l, d = 2, 9, 1002
    x = torch.randn(b, l, d, generator=seeded(40))
    y = torch.randn(b, l, d, generator=seeded(41)).to(BF)
    _, (sh, sc, g) = mods(b, d, 3, 42)
    with pytest.warns(RuntimeWarning, match="mod_in"):
        out = K.mod_in(x.to(dev), sh.to(dev), sc.to(dev), BF)
    close(out, S.mod_in(x, sh, sc, torch.float32))
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # once per segment: the second call is quiet
        K.mod_in(x.to(dev), sh.to(dev), sc.to(dev), BF)
    with pytest.warns(RuntimeWarning, match="gated_add_mod"):
        xo, h = K.gated_add_mod(x.to(dev), g.to(dev), y.to(dev), sh.to(dev), sc.to(dev), BF, False)
    rx, rh = S.gated_add_mod(x, g, y, sh, sc, torch.float32, False)
    assert torch.allclose(xo.cpu(), rx, rtol=1e-5, atol=1e-5)
    close(h, rh)
    with pytest.warns(RuntimeWarning, match="gated_add"):
        close(K.gated_add(x.to(dev), g.to(dev), y.to(dev), False), S.gated_add(x, g, y, False), 1e-5, 1e-5)
    # qkv rows starting 2 bytes into a buffer
    heads, dh, lq = 2, 64, 16
    base = torch.randn(1, lq, 3 * heads * dh + 1, generator=seeded(43)).to(BF)
    qkv = base[..., 1:]
    qs, ks = 1 + 0.02 * torch.randn(dh, generator=seeded(44)), 1 + 0.02 * torch.randn(dh, generator=seeded(45))
    cos, sin = S.rope_tables(torch.zeros(lq, 3), (16, 24, 24), 10000.0)
    qkv_dev = base.to(dev)[..., 1:]  # sliced on the GPU: a copy of the view would be aligned again
    assert qkv_dev.data_ptr() % 4 == 2
    with pytest.warns(RuntimeWarning, match="qkv_single"):
        q, k, v = K.qkv_single(qkv_dev, qs.to(dev), ks.to(dev), cos.to(dev), sin.to(dev), heads, BF)
    rq, rk, rv = S.qkv_single(qkv, qs, ks, cos, sin, heads, BF)
    close(q, rq)
    close(k, rk)
    assert torch.equal(v.cpu(), rv)
    # attn_mlp in fp32
    attn, mlp = torch.randn(1, 5, 64, generator=seeded(46)), torch.randn(1, 5, 96, generator=seeded(47))
    with pytest.warns(RuntimeWarning, match="attn_mlp"):
        o = K.attn_mlp(attn.to(dev), mlp.to(dev))
    close(o, S.attn_mlp(attn, mlp), 1e-5, 1e-5)
    # a bf16 residual stream (the kernels take fp32)
    xb = torch.randn(1, 4, 256, generator=seeded(48)).to(BF)
    _, (sh2, sc2, _) = mods(1, 256, 3, 49)
    close(K.mod_in(xb.to(dev), sh2.to(dev), sc2.to(dev), BF), S.mod_in(xb, sh2, sc2, BF))
    # argument errors are still errors
    with pytest.raises(ValueError):
        K.qkv_single(qkv_dev, qs[:5].to(dev), ks.to(dev), cos.to(dev), sin.to(dev), heads, BF)
