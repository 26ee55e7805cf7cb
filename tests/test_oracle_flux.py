"""Pins the block-composition oracle (oracle/flux.py) against vectors recorded from the reference.

tests/golden/flux_blocks_tiny.safetensors was written by tests/golden/make_golden.py
with selas's own double_block / single_block / final_layer / rope_tables on seeded
fp32 inputs (hidden 32, 2 heads, mlp 64, batch 2, 8 text + 16 image tokens).
"""

from __future__ import annotations

from pathlib import Path

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
