"""Pins the block-composition oracle (oracle/flux.py) against vectors recorded from the reference.

tests/golden/flux_blocks_tiny.safetensors was written by tests/golden/make_golden.py
with selas's own double_block / single_block / final_layer / rope_tables on seeded
fp32 inputs (hidden 32, 2 heads, mlp 64, batch 2, 8 text + 16 image tokens).
"""

from __future__ import annotations

from pathlib import Path

import pytest

import torch
from safetensors import safe_open

from oracle import flux as OF
from oracle import segments as S

GOLD = Path(__file__).resolve().parent / "golden" / "flux_blocks_tiny.safetensors"


def _load():
    with safe_open(str(GOLD), "pt") as f:
        meta = f.metadata()
        t = {k: f.get_tensor(k) for k in f.keys()}
    cfg = OF.FluxConfig(hidden=int(meta["hidden"]), heads=int(meta["heads"]), mlp_hidden=int(meta["mlp"]),
                        depth_double=1, depth_single=1, axes_dim=tuple(int(a) for a in meta["axes"].split(",")))
    units = {}
    for k, v in t.items():
        if k.startswith("w."):
            _, unit, name = k.split(".", 2)
            units.setdefault(unit, {})[name] = v
    return cfg, t, {u: OF.OracleUnit(w) for u, w in units.items()}


def test_rope_tables_match_reference():
    cfg, t, _ = _load()
    cos, sin = S.rope_tables(t["in.ids"], cfg.axes_dim, cfg.theta)
    assert torch.equal(cos, t["out.cos"]) and torch.equal(sin, t["out.sin"])


def test_blocks_match_reference_composition():
    cfg, t, u = _load()
    cos, sin = t["out.cos"], t["out.sin"]
    f32 = torch.float32
    img, txt = OF.double_block(u["double"], t["in.img"], t["in.txt"], t["in.dmod"], cos, sin, cfg, f32, False)
    assert torch.allclose(img, t["out.double.img"], atol=2e-5, rtol=1e-5)
    assert torch.allclose(txt, t["out.double.txt"], atol=2e-5, rtol=1e-5)
    x = torch.cat((t["in.txt"], t["in.img"]), dim=1)
    xo = OF.single_block(u["single"], x, t["in.smod"], cos, sin, cfg, f32, False)
    assert torch.allclose(xo, t["out.single.x"], atol=2e-5, rtol=1e-5)
    xg = OF.single_block(u["single"], x * 3e4, t["in.smod"], cos, sin, cfg, f32, True)
    assert torch.allclose(xg, t["out.single_guard.x"], rtol=1e-5, atol=1e-1)
    fin = OF.final_layer(u["globals"], t["in.img"], t["in.fmod"], f32)
    assert torch.allclose(fin, t["out.final"], atol=2e-5, rtol=1e-5)


def test_a_wrong_composition_is_caught():
    # planted mistake in the oracle side only: swapping the gates of the two residual updates
    cfg, t, u = _load()
    cos, sin = t["out.cos"], t["out.sin"]
    mod = t["in.dmod"].clone()
    d = cfg.hidden
    mod[:, 2 * d:3 * d], mod[:, 5 * d:6 * d] = t["in.dmod"][:, 5 * d:6 * d], t["in.dmod"][:, 2 * d:3 * d]
    img, _ = OF.double_block(u["double"], t["in.img"], t["in.txt"], mod, cos, sin, cfg, torch.float32, False)
    assert not torch.allclose(img, t["out.double.img"], atol=1e-3)


def test_bf16_blocks_match_reference_casts():
    # The reference's blocks in the bf16 compute dtype (weights decoded to bf16, segments casting where
    # flux.py:164-200 casts, F.linear in bf16 on the CPU). The oracle's bf16 linears (bf16 operands, fp32
    # accumulation, one rounding) match them except where a rounding lands the other way: the updates
    # agree to well inside the 4e-3 path tolerance, and a wrong cast (the fp32 oracle) does not.
    cfg, t, u = _load()
    cos, sin = t["out.cos"], t["out.sin"]
    bf16 = torch.bfloat16
    ub = {k: OF.OracleUnit(v.t, bf16) for k, v in u.items()}

    def rel(a, b):
        return ((a.double() - b.double()).norm() / b.double().norm()).item()

    img, txt = OF.double_block(ub["double"], t["in.img"], t["in.txt"], t["in.dmod"].to(bf16), cos, sin, cfg, bf16,
                               False)
    ri, rt = t["out.bf16.double.img"], t["out.bf16.double.txt"]
    assert rel(img - t["in.img"], ri - t["in.img"]) < 2e-3 and rel(txt - t["in.txt"], rt - t["in.txt"]) < 2e-3
    x = torch.cat((t["in.txt"], t["in.img"]), dim=1)
    xo = OF.single_block(ub["single"], x, t["in.smod"].to(bf16), cos, sin, cfg, bf16, False)
    assert rel(xo - x, t["out.bf16.single.x"] - x) < 2e-3
    fin = OF.final_layer(ub["globals"], t["in.img"], t["in.fmod"].to(bf16), bf16)
    assert rel(fin, t["out.bf16.final"]) < 4e-3
    # the fp32 composition is measurably further from the bf16 golden than the bf16 oracle is
    img32, _ = OF.double_block(u["double"], t["in.img"], t["in.txt"], t["in.dmod"].to(bf16).float(), cos, sin, cfg,
                               torch.float32, False)
    assert rel(img32 - t["in.img"], ri - t["in.img"]) > 2 * rel(img - t["in.img"], ri - t["in.img"])


RUNNER = Path(__file__).resolve().parent / "golden" / "flux_runner_tiny.safetensors"


def _runner():
    with safe_open(str(RUNNER), "pt") as f:
        meta = f.metadata()
        t = {k: f.get_tensor(k) for k in f.keys()}
    cfg = OF.FluxConfig(hidden=int(meta["hidden"]), heads=int(meta["heads"]), mlp_hidden=int(meta["mlp"]),
                        depth_double=int(meta["double"]), depth_single=int(meta["single"]), in_channels=64,
                        context_dim=int(meta["context"]), vec_dim=int(meta["vec"]),
                        axes_dim=tuple(int(a) for a in meta["axes"].split(",")))
    units = {}
    for k, v in t.items():
        if k.startswith("w."):
            rest = k[2:]
            unit = "globals" if rest.startswith("globals.") else ".".join(rest.split(".")[:2])
            if rest.split(".")[2:3] == ["mod"]:
                unit += ".mod"
            units.setdefault(unit, {})[rest[len(unit) + 1:]] = v
    return cfg, t, {n: OF.OracleUnit(w) for n, w in units.items()}


def _runner_parts(cfg, u):
    doubles = [u[f"double.{i}"] for i in range(cfg.depth_double)]
    singles = [u[f"single.{i}"] for i in range(cfg.depth_single)]
    mods = [u[f"double.{i}.mod"] for i in range(cfg.depth_double)] + \
        [u[f"single.{i}.mod"] for i in range(cfg.depth_single)]
    return doubles, singles, mods


def test_timestep_embedding_and_svec_match_reference():
    cfg, t, u = _runner()
    sig = t["in.sigmas"].tolist()
    temb = S.timestep_embedding(torch.tensor(sig[:-1], dtype=torch.float32), 256)
    assert torch.allclose(temb, t["out.temb"], atol=1e-6, rtol=0)
    assert torch.allclose(OF.mlp_embed(u["globals"], "time_in", temb), t["out.time_mlp"], atol=2e-5, rtol=1e-5)
    for i in range(t["in.pooled"].shape[0]):
        sv = OF.svec(u["globals"], cfg, sig, float(t["in.guidance"]), t["in.pooled"][i:i + 1], torch.float32)
        assert sv.shape == (len(sig) - 1, 1, cfg.hidden)
        assert torch.allclose(sv, t[f"out.svec{i}"], atol=2e-5, rtol=1e-5)


def test_modulations_prepare_and_steps_match_reference():
    cfg, t, u = _runner()
    doubles, singles, mod_units = _runner_parts(cfg, u)
    sig = t["in.sigmas"].tolist()
    g = float(t["in.guidance"])
    pooled = t["in.pooled"]
    svecs = [OF.svec(u["globals"], cfg, sig, g, pooled[i:i + 1], torch.float32) for i in range(pooled.shape[0])]
    per_image = OF.modulations(mod_units, svecs, cfg.depth_double)
    mods = [torch.cat([p[j] for p in per_image], dim=1) for j in range(len(mod_units))]
    names = [f"double.{i}" for i in range(cfg.depth_double)] + [f"single.{i}" for i in range(cfg.depth_single)]
    for n, m in zip(names, mods):
        assert torch.allclose(m, t[f"out.mods.{n}"], atol=2e-5, rtol=1e-5), n
    cond = OF.prepare(u["globals"], cfg, sig, g, pooled, t["in.txt"], t["in.img_ids"], t["in.txt_ids"], mods,
                      torch.float32)
    assert torch.allclose(cond.final_mod, t["out.final_mod"], atol=2e-5, rtol=1e-5)
    assert torch.allclose(cond.txt, t["out.txt"], atol=2e-5, rtol=1e-5)
    assert torch.equal(cond.cos, t["out.cos"]) and torch.equal(cond.sin, t["out.sin"])
    x = t["in.latents"]
    for s in range(2):
        pred = OF.step(u["globals"], doubles, singles, cfg, s, x, cond, torch.float32)
        assert torch.allclose(pred, t[f"out.step{s}.pred"], atol=5e-5, rtol=1e-4)
        x = OF.euler(x, sig, s, pred)
        assert torch.allclose(x, t[f"out.step{s}.x"], atol=5e-5, rtol=1e-4)


def test_planted_mistakes_in_the_runner_are_caught():
    # oracle-side plants: text before image swapped in the modulation concat; the Euler step's sign
    cfg, t, u = _runner()
    _, _, mod_units = _runner_parts(cfg, u)
    sig = t["in.sigmas"].tolist()
    sv = OF.svec(u["globals"], cfg, sig, float(t["in.guidance"]), t["in.pooled"][:1], torch.float32)
    w = mod_units[0]
    swapped = torch.cat((w.linear(sv, "txt_mod.lin"), w.linear(sv, "img_mod.lin")), dim=-1)
    assert not torch.allclose(swapped, t["out.mods.double.0"][:, :1], atol=1e-3)
    pred = t["out.step0.pred"]
    wrong = t["in.latents"] - (sig[1] - sig[0]) * pred
    assert not torch.allclose(wrong, t["out.step0.x"], atol=1e-3)
    with pytest.raises(FloatingPointError):
        OF.euler(t["in.latents"], sig, 0, pred * float("inf"))


def test_unit_flops_matches_the_published_totals():
    # docs/PLAN.md:51-52: 59.5 T linear + 14.9 T attention per step at 1024^2 (4096 image + 512 text
    # tokens), 19.8 T + 1.7 T at 512^2 (1024 + 512), over 19 double and 38 single blocks.
    cfg = OF.FluxConfig()
    for li, lin_t, att_t in ((4096, 59.5, 14.9), (1024, 19.8, 1.7)):
        lin = sum(OF.unit_flops(k, cfg, li, 512, 1)[0] * n for k, n in (("double", 19), ("single", 38)))
        att = sum(OF.unit_flops(k, cfg, li, 512, 1)[1] * n for k, n in (("double", 19), ("single", 38)))
        assert round(lin / 1e12, 1) == lin_t and round(att / 1e12, 1) == att_t
    # a block's linear count is 2 * tokens * its weight count (113,246,208 for FLUX-dev, both kinds),
    # and it scales with the batch
    assert OF.unit_flops("double", cfg, 4096, 512, 1)[0] == 2 * 4608 * 113_246_208
    assert OF.unit_flops("single", cfg, 4096, 512, 3)[0] == 3 * 2 * 4608 * 113_246_208
    assert OF.unit_flops("globals", cfg, 4096, 512, 1) == (0.0, 0.0)


def test_product_runner_helpers_match_reference_vectors():
    # selas_amd.flux's own schedule, position ids, timestep embedding and RoPE tables (the values its GPU
    # runner is fed) against what selas's sampling.py / flux.py produced for the tiny runner: 3 steps over
    # 16 image tokens, a 4 x 4 latent grid (64 x 64 pixels in selas's image_ids), 8 text tokens.
    import math

    from selas_amd import flux as PF

    cfg, t, _ = _runner()
    sig = PF.get_schedule(len(t["in.sigmas"]) - 1, 16)
    assert torch.equal(torch.tensor(sig, dtype=torch.float64), t["in.sigmas"])
    img_ids, txt_ids = PF.image_ids(4, 4), PF.text_ids(8)
    assert torch.equal(img_ids, t["in.img_ids"]) and torch.equal(txt_ids, t["in.txt_ids"])
    temb = PF.timestep_embedding(torch.tensor(sig[:-1], dtype=torch.float32), 256)
    assert torch.allclose(temb, t["out.temb"], atol=1e-6, rtol=0)
    cos, sin = PF.rope_tables(torch.cat((txt_ids, img_ids)), cfg.axes_dim, cfg.theta)
    assert torch.equal(cos, t["out.cos"]) and torch.equal(sin, t["out.sin"])
    # The shift at FLUX's own sizes, from its closed form: mu = 0.5 + 0.65 (L - 256) / 3840, so L = 4096
    # (1024^2) gives mu = 1.15 and sigma(t) = e^mu / (e^mu + 1/t - 1); L = 1024 (512^2) mu = 0.63.
    for seq, mu in ((4096, 1.15), (1024, 0.5 + 0.65 * 768 / 3840)):
        s = PF.get_schedule(28, seq)
        assert s[0] == 1.0 and s[-1] == 0.0 and len(s) == 29
        for i in (7, 14, 21):
            tt = 1 - i / 28
            assert abs(s[i] - math.exp(mu) / (math.exp(mu) + 1 / tt - 1)) < 1e-12
    assert PF.get_schedule(4, 4096, shift=False) == [1.0, 0.75, 0.5, 0.25, 0.0]
    # rows are (0, row, col): the last image token of a 64 x 48 grid sits at row 63, column 47
    ids = PF.image_ids(64, 48)
    assert ids.shape == (3072, 3) and ids[-1].tolist() == [0.0, 63.0, 47.0] and ids[48].tolist() == [0.0, 1.0, 0.0]
