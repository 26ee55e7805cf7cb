"""FLUX blocks on the GPU (fused NF4 linears + segment kernels + fused attention) against the oracle blocks
on the CPU with the same decoded NF4 operands and the reference's bf16 arithmetic (oracle/flux.py, pinned
by goldens the reference's own functions wrote, in fp32 and in bf16).

Tolerance: block outputs are compared on the residual update (out - in) at relative L2 <= 4e-3, the
path's tolerance; the step's velocity likewise.
"""

from __future__ import annotations

import pytest
import torch

from oracle import flux as OF
from oracle import segments as S
from selas_amd import flux as F

from .conftest import seeded

pytestmark = pytest.mark.gpu

CFG = F.FluxConfig(hidden=256, heads=2, mlp_hidden=1024, depth_double=2, depth_single=2, in_channels=64,
                   context_dim=128, vec_dim=64, axes_dim=(16, 56, 56))
OCFG = OF.FluxConfig(hidden=256, heads=2, mlp_hidden=1024, depth_double=2, depth_single=2, in_channels=64,
                     context_dim=128, vec_dim=64, axes_dim=(16, 56, 56))


BF16 = torch.bfloat16
L2 = 4e-3


def oracle_unit(view):
    enc = {n: (e.codec, e.shape, e.meta, {k: v.cpu() for k, v in e.parts.items()}) for n, e in view.tensors.items()}
    return OF.OracleUnit.from_encoded(enc, BF16)


def rel(a, b):
    return ((a.double().cpu() - b.double()).norm() / b.double().norm()).item()


@pytest.fixture(scope="module")
def model():
    return F.RandomFlux(CFG, "cuda", torch.bfloat16, seed=3)


def inputs(b, lt, grid):
    g = seeded(21)
    li = grid * grid
    img = torch.randn(b, li, CFG.hidden, generator=g)
    txt = torch.randn(b, lt, CFG.hidden, generator=g)
    ids = torch.cat((torch.zeros(lt, 3), F.image_ids(grid, grid)), dim=0)
    cos, sin = S.rope_tables(ids, CFG.axes_dim, CFG.theta)
    return img, txt, cos, sin


def test_double_block(model):
    img, txt, cos, sin = inputs(2, 64, 8)
    mod = (torch.randn(2, 12 * CFG.hidden, generator=seeded(22)) * 0.3).to(torch.bfloat16)
    dev = torch.device("cuda")
    gi, gt = F.double_block(model.doubles[0], img.to(dev), txt.to(dev), mod.to(dev), cos.to(dev), sin.to(dev), CFG,
                            torch.bfloat16, False)
    ri, rt = OF.double_block(oracle_unit(model.doubles[0]), img, txt, mod, cos, sin, OCFG, BF16, False)
    assert rel(gi - img.cuda(), ri - img) < L2 and rel(gt - txt.cuda(), rt - txt) < L2


def test_single_block(model):
    img, txt, cos, sin = inputs(1, 64, 8)
    x = torch.cat((txt, img), dim=1)
    mod = (torch.randn(1, 3 * CFG.hidden, generator=seeded(23)) * 0.3).to(torch.bfloat16)
    dev = torch.device("cuda")
    gx = F.single_block(model.singles[0], x.to(dev), mod.to(dev), cos.to(dev), sin.to(dev), CFG, torch.bfloat16,
                        False)
    rx = OF.single_block(oracle_unit(model.singles[0]), x, mod, cos, sin, OCFG, BF16, False)
    assert rel(gx - x.cuda(), rx - x) < L2


def test_modulations_and_step(model):
    # hoisted modulation GEMVs (M = steps = 5) and one step through 2 double + 2 single blocks
    dev = torch.device("cuda")
    sv = torch.nn.functional.silu(torch.randn(5, 1, CFG.hidden, generator=seeded(24))).to(torch.bfloat16)
    mods = model.modulations(sv.to(dev))
    units = [oracle_unit(u) for u in model.mods]
    for i, (m, u) in enumerate(zip(mods, units)):
        if i < len(model.doubles):
            ref = torch.cat((u.linear(sv, "img_mod.lin"), u.linear(sv, "txt_mod.lin")), dim=-1)
        else:
            ref = u.linear(sv, "modulation.lin")
        assert m.shape == ref.shape and rel(m, ref) < L2
    img, txt, cos, sin = inputs(1, 64, 8)
    lat = torch.randn(1, 64, 64, generator=seeded(25))
    fmod = (torch.randn(1, 2 * CFG.hidden, generator=seeded(26)) * 0.3).to(torch.bfloat16)
    s = 2
    out = model.step(lat.to(dev), txt.to(dev), [m[s] for m in mods], fmod.to(dev), cos.to(dev), sin.to(dev))
    g = oracle_unit(model.globals)
    x_img = g.linear(lat.to(BF16), "img_in").float()
    t = txt
    for i, w in enumerate(model.doubles):
        x_img, t = OF.double_block(oracle_unit(w), x_img, t, mods[i][s].cpu(), cos, sin, OCFG, BF16, False)
    x = torch.cat((t, x_img), dim=1)
    for j, w in enumerate(model.singles):
        x = OF.single_block(oracle_unit(w), x, mods[len(model.doubles) + j][s].cpu(), cos, sin, OCFG, BF16, False)
    ref = OF.final_layer(g, x[:, 64:], fmod, BF16)
    assert out.shape == (1, 64, 64) and torch.isfinite(out).all()
    assert rel(out, ref) < L2


def test_batched_step_equals_images_one_by_one(model):
    # C5 runs batch 4 at 512^2: each image brings its own modulations, and every kernel on the path
    # works per token (linears, segments) or per (image, head) (attention), so a batched step must
    # give each image the velocity it gets alone.
    dev = torch.device("cuda")
    g = seeded(27)
    b = 3
    mods = [model.modulations(torch.nn.functional.silu(torch.randn(4, 1, CFG.hidden, generator=g)).to(torch.bfloat16)
                              .to(dev)) for _ in range(b)]
    _, txt, cos, sin = inputs(b, 64, 8)
    lat = torch.randn(b, 64, 64, generator=g)
    fmod = (torch.randn(b, 2 * CFG.hidden, generator=g) * 0.3).to(torch.bfloat16)
    s = 1
    args = (cos.to(dev), sin.to(dev))
    out = model.step(lat.to(dev), txt.to(dev), [torch.cat([m[j][s] for m in mods], dim=0) for j in range(len(mods[0]))],
                     fmod.to(dev), *args)
    assert out.shape == (b, 64, 64) and torch.isfinite(out).all()
    for i in range(b):
        one = model.step(lat[i:i + 1].to(dev), txt[i:i + 1].to(dev), [m[s] for m in mods[i]], fmod[i:i + 1].to(dev),
                         *args)
        assert rel(out[i:i + 1], one.cpu()) < 1e-3


def test_chained_blocks_equal_separate_segments(model, monkeypatch):
    # RandomFlux.step runs each block's closing residual add together with the next block's mod_in
    # (gated_add_mod); the velocity must be bit for bit that of the separate gated_add + mod_in kernels.
    dev = torch.device("cuda")
    g = seeded(30)
    mods = model.modulations(torch.nn.functional.silu(torch.randn(3, 2, CFG.hidden, generator=g))
                             .to(torch.bfloat16).to(dev))
    _, txt, cos, sin = inputs(2, 64, 8)
    lat = torch.randn(2, 64, 64, generator=g)
    fmod = (torch.randn(2, 2 * CFG.hidden, generator=g) * 0.3).to(torch.bfloat16)

    def run():
        return model.step(lat.to(dev), txt.to(dev), [m[1] for m in mods], fmod.to(dev), cos.to(dev), sin.to(dev))

    chained = run()
    monkeypatch.setattr(F, "CHAIN_BLOCKS", False)
    separate = run()
    assert torch.isfinite(chained).all() and torch.equal(chained, separate)


def test_fused_gelu_blocks_equal_composed_blocks(model, monkeypatch):
    # linear1 / mlp.0 with GELU in the GEMM epilogue, written into linear2's input next to the attention
    # output, against the unfused sequence (linear, GELU kernel, attention, concat): bit for bit.
    img, txt, cos, sin = inputs(2, 64, 8)
    dev = torch.device("cuda")
    img, txt, cos, sin = img.to(dev), txt.to(dev), cos.to(dev), sin.to(dev)
    dmod = (torch.randn(2, 12 * CFG.hidden, generator=seeded(28)) * 0.3).to(torch.bfloat16).to(dev)
    smod = (torch.randn(2, 3 * CFG.hidden, generator=seeded(29)) * 0.3).to(torch.bfloat16).to(dev)
    x = torch.cat((txt, img), dim=1)

    def run():
        d = F.double_block(model.doubles[1], img, txt, dmod, cos, sin, CFG, torch.bfloat16, False)
        return d + (F.single_block(model.singles[1], x, smod, cos, sin, CFG, torch.bfloat16, False),)

    fused = run()
    monkeypatch.setattr(F, "_fused_gelu", lambda w, k: False)
    composed = run()
    for a, b in zip(fused, composed):
        assert torch.equal(a, b)


def test_int8_row_blocks(monkeypatch):
    # The same blocks with int8_row weights (selas convert --quant int8): fused int8 GEMMs, GELU
    # epilogue and skinny modulation linears, against the oracle decoding the same q and scales.
    m8 = F.RandomFlux(CFG, "cuda", torch.bfloat16, seed=5, n_double=1, n_single=1, quant="int8")
    assert m8.doubles[0].codec("img_mlp.0.weight") == "int8_row"
    dev = torch.device("cuda")
    img, txt, cos, sin = inputs(2, 64, 8)
    mod = (torch.randn(2, 12 * CFG.hidden, generator=seeded(30)) * 0.3).to(torch.bfloat16)
    gi, gt = F.double_block(m8.doubles[0], img.to(dev), txt.to(dev), mod.to(dev), cos.to(dev), sin.to(dev), CFG,
                            torch.bfloat16, False)
    ri, rt = OF.double_block(oracle_unit(m8.doubles[0]), img, txt, mod, cos, sin, OCFG, BF16, False)
    assert rel(gi - img.cuda(), ri - img) < L2 and rel(gt - txt.cuda(), rt - txt) < L2
    x = torch.cat((txt, img), dim=1)
    smod = (torch.randn(2, 3 * CFG.hidden, generator=seeded(31)) * 0.3).to(torch.bfloat16)
    gx = F.single_block(m8.singles[0], x.to(dev), smod.to(dev), cos.to(dev), sin.to(dev), CFG, torch.bfloat16, False)
    rx = OF.single_block(oracle_unit(m8.singles[0]), x, smod, cos, sin, OCFG, BF16, False)
    assert rel(gx - x.cuda(), rx - x) < L2
    sv = torch.nn.functional.silu(torch.randn(5, 1, CFG.hidden, generator=seeded(32))).to(torch.bfloat16)
    mods = m8.modulations(sv.to(dev))
    u = oracle_unit(m8.mods[1])
    assert rel(mods[1], u.linear(sv, "modulation.lin")) < L2
    fused = F.single_block(m8.singles[0], x.to(dev), smod.to(dev), cos.to(dev), sin.to(dev), CFG, torch.bfloat16,
                           False)
    monkeypatch.setattr(F, "_fused_gelu", lambda w, k: False)
    composed = F.single_block(m8.singles[0], x.to(dev), smod.to(dev), cos.to(dev), sin.to(dev), CFG, torch.bfloat16,
                              False)
    assert torch.equal(fused, composed)


def test_planner_measurements(dev):
    from selas_amd import planner as P

    prof = P.measure_profile(dev)
    assert prof.measured == ("attn_flops", "dequant_bw", "matmul_flops")
    assert 2e14 < prof.matmul_flops < 2.5e15 and 2e14 < prof.attn_flops < 2.5e15 and 2e11 < prof.dequant_bw < 8e12


def test_blocks_at_a_token_count_off_the_tiles(model):
    # 60 text + 7 x 7 image tokens = 109: attention's last key and query tiles are partial.
    img, txt, cos, sin = inputs(1, 60, 7)
    dev = torch.device("cuda")
    x = torch.cat((txt, img), dim=1)
    mod = (torch.randn(1, 3 * CFG.hidden, generator=seeded(33)) * 0.3).to(torch.bfloat16)
    gx = F.single_block(model.singles[1], x.to(dev), mod.to(dev), cos.to(dev), sin.to(dev), CFG, torch.bfloat16,
                        False)
    rx = OF.single_block(oracle_unit(model.singles[1]), x, mod, cos, sin, OCFG, BF16, False)
    assert rel(gx - x.cuda(), rx - x) < L2
    dmod = (torch.randn(1, 12 * CFG.hidden, generator=seeded(34)) * 0.3).to(torch.bfloat16)
    gi, gt = F.double_block(model.doubles[1], img.to(dev), txt.to(dev), dmod.to(dev), cos.to(dev), sin.to(dev), CFG,
                            torch.bfloat16, False)
    ri, rt = OF.double_block(oracle_unit(model.doubles[1]), img, txt, dmod, cos, sin, OCFG, BF16, False)
    assert rel(gi - img.cuda(), ri - img) < L2 and rel(gt - txt.cuda(), rt - txt) < L2
