"""Writes golden vectors for the FLUX block composition with the reference's own functions.

Run in the build container (where the reference is mounted):
    python tests/golden/make_golden.py /root/reference

What it pins: the order in which selas's double_block / single_block /
final_layer (selas/models/flux.py:300-343) chain modulation, linears, head
split, QK-norm, RoPE, attention and gated residuals, and rope_tables
(flux.py:106-114) on text + image position ids (selas/sampling.py:58-69).
No closed form or reference test pins these, so they are recorded from the
reference code itself, on seeded random fp32 inputs and weights, with eager
segments on the CPU in fp32. Only inputs and outputs are stored (a
safetensors file next to this script); nothing of the reference is copied.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

OUT = Path(__file__).resolve().parent / "flux_blocks_tiny.safetensors"

# A small FLUX-shaped config: hidden 32, 2 heads of 16 (RoPE axes 4+6+6), mlp 64.
HIDDEN, HEADS, MLP, AXES = 32, 2, 64, (4, 6, 6)
BATCH, LT, GRID = 2, 8, 4  # 8 text tokens, 4x4 image tokens


class DenseView:
    """Minimal stand-in for selas.store.UnitView over plain fp32 tensors."""

    def __init__(self, tensors):
        self.t = tensors

    def get(self, name, dtype=None):
        return self.t[name].to(dtype or torch.float32)

    def linear(self, x, prefix, dtype=None):
        b = self.t.get(prefix + ".bias")
        return torch.nn.functional.linear(x, self.t[prefix + ".weight"], b)


def _lin(sd, g, name, i, o):
    sd[name + ".weight"] = torch.randn(o, i, generator=g) / math.sqrt(i)
    sd[name + ".bias"] = torch.randn(o, generator=g) * 0.02


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from selas.models.flux import EAGER, FluxConfig, double_block, final_layer, rope_tables, single_block
    from selas.sampling import image_ids, text_ids

    cfg = FluxConfig(hidden=HIDDEN, heads=HEADS, mlp_hidden=MLP, depth_double=1, depth_single=1, axes_dim=AXES)
    g = torch.Generator().manual_seed(1234)
    d, m = HIDDEN, MLP
    dbl, sgl, glb = {}, {}, {}
    for s in ("img", "txt"):
        _lin(dbl, g, f"{s}_attn.qkv", d, 3 * d)
        _lin(dbl, g, f"{s}_attn.proj", d, d)
        _lin(dbl, g, f"{s}_mlp.0", d, m)
        _lin(dbl, g, f"{s}_mlp.2", m, d)
        for q in ("query", "key"):
            dbl[f"{s}_attn.norm.{q}_norm.scale"] = 1 + 0.1 * torch.randn(d // HEADS, generator=g)
    _lin(sgl, g, "linear1", d, 3 * d + m)
    _lin(sgl, g, "linear2", d + m, d)
    for q in ("query", "key"):
        sgl[f"norm.{q}_norm.scale"] = 1 + 0.1 * torch.randn(d // HEADS, generator=g)
    _lin(glb, g, "final_layer.linear", d, 64)

    li = GRID * GRID
    img = torch.randn(BATCH, li, d, generator=g)
    txt = torch.randn(BATCH, LT, d, generator=g)
    dmod = torch.randn(BATCH, 12 * d, generator=g) * 0.3
    smod = torch.randn(BATCH, 3 * d, generator=g) * 0.3
    fmod = torch.randn(BATCH, 2 * d, generator=g) * 0.3
    # image_ids takes pixel sizes: 16 px per packed latent token.
    ids = torch.cat((text_ids(LT), image_ids(16 * GRID, 16 * GRID)), dim=0)
    ids[:LT, 0] = torch.arange(LT, dtype=ids.dtype) * 0.5  # nonzero text positions exercise axis 0 too
    cos, sin = rope_tables(ids, AXES, 10000.0)

    f32 = torch.float32
    with torch.no_grad():
        img_o, txt_o = double_block(DenseView(dbl), img, txt, dmod, cos, sin, cfg, f32, False, EAGER)
        x = torch.cat((txt, img), dim=1)
        x_o = single_block(DenseView(sgl), x, smod, cos, sin, cfg, f32, False, EAGER)
        x_g = single_block(DenseView(sgl), x * 3e4, smod, cos, sin, cfg, f32, True, EAGER)
        fin = final_layer(DenseView(glb), img, fmod, f32, EAGER)

    tensors = {"in.img": img, "in.txt": txt, "in.dmod": dmod, "in.smod": smod, "in.fmod": fmod, "in.ids": ids,
               "out.cos": cos, "out.sin": sin, "out.double.img": img_o, "out.double.txt": txt_o,
               "out.single.x": x_o, "out.single_guard.x": x_g, "out.final": fin}
    tensors.update({f"w.double.{k}": v for k, v in dbl.items()})
    tensors.update({f"w.single.{k}": v for k, v in sgl.items()})
    tensors.update({f"w.globals.{k}": v for k, v in glb.items()})
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(OUT),
              metadata={"hidden": str(HIDDEN), "heads": str(HEADS), "mlp": str(MLP), "axes": ",".join(map(str, AXES)),
                        "batch": str(BATCH), "lt": str(LT), "grid": str(GRID)})
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
