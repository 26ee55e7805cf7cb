"""Pins the segment oracle (oracle/segments.py) against library routines, closed forms and invariants."""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import segments as S

from .conftest import seeded


def test_layernorm_matches_torch_layer_norm_and_invariants():
    x = torch.randn(6, 3072, generator=seeded(0), dtype=torch.float64) * 3 + 1
    ours = S.ln(x)
    ref = F.layer_norm(x, (3072,), eps=1e-6)  # a library routine
    assert torch.allclose(ours, ref, atol=1e-12, rtol=0)
    assert torch.allclose(ours.mean(-1), torch.zeros(6, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(ours.pow(2).mean(-1), torch.ones(6, dtype=torch.float64), atol=1e-6)


def test_mod_in_modulation_closed_forms():
    x = torch.randn(1, 5, 64, generator=seeded(1))
    shift = torch.randn(1, 1, 64, generator=seeded(2))
    # scale == -1 cancels the normalised input: the output is the shift exactly
    out = S.mod_in(x, shift, -torch.ones(1, 1, 64), torch.float32)
    assert torch.equal(out, shift.expand(1, 5, 64))
    # scale == 0, shift == 0 is plain LayerNorm
    out = S.mod_in(x, torch.zeros(1, 1, 64), torch.zeros(1, 1, 64), torch.float32)
    assert torch.allclose(out, F.layer_norm(x, (64,), eps=1e-6), atol=1e-6)


def test_gated_add_and_fp16_guard():
    x = torch.zeros(1, 1, 4)
    g = torch.full((1, 1, 4), 2.0)
    y = torch.tensor([[[1.0, -1e6, 1e6, float("nan")]]])
    out = S.gated_add(x, g, y, True)
    assert out[0, 0, 0] == 2.0 and out[0, 0, 1] == -2 * 65504.0 and out[0, 0, 2] == 2 * 65504.0
    assert torch.isnan(out[0, 0, 3])  # the clamp does not swallow NaN
    assert S.gated_add(x, g, y, False)[0, 0, 1] == -2e6


def test_rms_norm_unit_rms_and_scale():
    x = torch.randn(2, 3, 7, 128, generator=seeded(3)) * 5
    scale = 1 + 0.1 * torch.randn(128, generator=seeded(4))
    out = S.qk_rms(x, torch.ones(128))
    assert torch.allclose(out.pow(2).mean(-1), torch.ones(2, 3, 7), atol=1e-4)
    assert torch.allclose(S.qk_rms(x, scale), out * scale, atol=1e-6)


def test_rope_is_complex_rotation_and_relative():
    x = torch.randn(1, 2, 9, 16, generator=seeded(5), dtype=torch.float64)
    ang = torch.rand(9, 8, generator=seeded(6), dtype=torch.float64) * 6
    out = S.apply_rope(x, ang.cos(), ang.sin())
    z = torch.complex(x[..., 0::2], x[..., 1::2]) * torch.exp(1j * ang)  # textbook: rotate each pair
    assert torch.allclose(out[..., 0::2], z.real, atol=1e-12) and torch.allclose(out[..., 1::2], z.imag, atol=1e-12)
    assert torch.allclose(out.norm(dim=-1), x.norm(dim=-1), atol=1e-12)
    # relative position: <R(p)q, R(p')k> depends only on p - p'
    freqs = torch.rand(8, generator=seeded(7), dtype=torch.float64)
    q, k = x[0, 0, 0], x[0, 1, 0]

    def rot(v, p):
        a = p * freqs
        return S.apply_rope(v[None], a.cos()[None], a.sin()[None])[0]

    assert abs(rot(q, 5.0) @ rot(k, 2.0) - rot(q, 13.0) @ rot(k, 10.0)) < 1e-10


def test_rope_tables_closed_forms():
    axes = (16, 56, 56)
    ids = torch.tensor([[0.0, 0.0, 0.0], [0.0, 3.0, 7.0], [2.0, 0.0, 1.0]])
    cos, sin = S.rope_tables(ids, axes, 10000.0)
    assert cos.shape == (3, 64) and cos.dtype == torch.float32
    assert torch.equal(cos[0], torch.ones(64)) and torch.equal(sin[0], torch.zeros(64))
    # first frequency of each axis is theta^0 = 1: the angle is the position itself
    assert cos[1, 8] == torch.tensor(math.cos(3.0), dtype=torch.float64).float()
    assert sin[1, 36] == torch.tensor(math.sin(7.0), dtype=torch.float64).float()
    assert cos[2, 0] == torch.tensor(math.cos(2.0), dtype=torch.float64).float()
    # frequency j of an axis of width d is theta^(-2j/d)
    j, d = 5, 56
    want = math.sin(7.0 * 10000.0 ** (-2 * j / d))
    assert abs(sin[1, 8 + 28 + j].item() - want) < 1e-7


def test_gelu_matches_torch():
    h = torch.randn(4, 1000, generator=seeded(8)) * 4
    assert torch.allclose(S.gelu(h), F.gelu(h, approximate="tanh"), atol=1e-6)
    hb = h.to(torch.bfloat16)
    ours, ref = S.gelu(hb).float(), F.gelu(hb.float(), approximate="tanh").to(torch.bfloat16).float()
    assert (ours != ref).float().mean() < 1e-2  # at most rare one-ulp tie differences after the bf16 rounding


def test_head_split_by_one_hot_probes():
    H, Dh, L = 3, 8, 2
    for which, head, d in [(0, 0, 0), (1, 2, 5), (2, 1, 7)]:
        qkv = torch.zeros(1, L, 3 * H * Dh)
        qkv[0, 1, which * H * Dh + head * Dh + d] = 1.0
        parts = S.heads(qkv, H)
        for w in range(3):
            nz = parts[w].nonzero().tolist()
            assert nz == ([[0, head, 1, d]] if w == which else [])
    # after RMSNorm a one-hot head becomes sqrt(Dh) * scale at that position
    qkv = torch.zeros(1, 1, 3 * H * Dh)
    qkv[0, 0, 1 * Dh + 3] = 2.0
    q, _, _ = S.qkv_single(qkv, torch.ones(Dh), torch.ones(Dh), torch.ones(1, Dh // 2), torch.zeros(1, Dh // 2), H,
                           torch.float32)
    assert abs(q[0, 1, 0, 3].item() - math.sqrt(Dh)) < 1e-4


def test_qkv_double_joins_text_first():
    H, Dh, Lt, Li = 2, 8, 3, 4
    t = torch.randn(1, Lt, 3 * H * Dh, generator=seeded(9))
    i = torch.randn(1, Li, 3 * H * Dh, generator=seeded(10))
    one = torch.ones(Dh)
    cos, sin = torch.ones(Lt + Li, Dh // 2), torch.zeros(Lt + Li, Dh // 2)
    q, k, v = S.qkv_double(t, i, one, one, one * 2, one, cos, sin, H, torch.float32)
    assert torch.equal(v[:, :, :Lt], S.heads(t, H)[2]) and torch.equal(v[:, :, Lt:], S.heads(i, H)[2])
    assert torch.allclose(q[:, :, Lt:], 2 * S.qk_rms(S.heads(i, H)[0], one), atol=1e-6)


def test_attn_mlp_concat_order():
    a = torch.randn(1, 3, 4, generator=seeded(11))
    m = torch.randn(1, 3, 6, generator=seeded(12))
    out = S.attn_mlp(a, m)
    assert torch.equal(out[..., :4], a) and torch.allclose(out[..., 4:], F.gelu(m, approximate="tanh"), atol=1e-6)


def test_timestep_embedding_closed_form():
    t = torch.tensor([0.0, 0.5])
    emb = S.timestep_embedding(t, 8)
    assert torch.equal(emb[0], torch.tensor([1.0] * 4 + [0.0] * 4))
    freqs = np.exp(-math.log(10000.0) * np.arange(4) / 4)
    assert np.allclose(emb[1, :4].numpy(), np.cos(500.0 * freqs), atol=1e-4)
