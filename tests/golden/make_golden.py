"""Writes golden vectors for the FLUX composition with the reference's own functions.

Run in the build container (where the reference is mounted):
    python tests/golden/make_golden.py /root/reference

What it pins:
  flux_blocks_tiny.safetensors: the order in which selas's double_block /
    single_block / final_layer (selas/models/flux.py:300-343) chain modulation,
    linears, head split, QK-norm, RoPE, attention and gated residuals, in fp32
    and in bf16 (the casts to the compute dtype where the reference casts),
    and rope_tables (flux.py:106-114) on text + image position ids
    (selas/sampling.py:58-69);
  flux_runner_tiny.safetensors: FluxRunner's prologue and step on a two-double,
    two-single-block model: timestep_embedding (flux.py:95-103), mlp_embed
    (150-151), svec (411-425), modulations (428-445), prepare (448-465) and
    two steps (527-582) with the Euler update of selas/pipeline.py:489.
No closed form or reference test pins these, so they are recorded from the
reference code itself, on seeded random inputs and weights, with eager
segments on the CPU. Only inputs and outputs are stored (safetensors files
next to this script); nothing of the reference is copied. FluxRunner is driven
through minimal stand-ins for its weight store (DenseView for UnitView, a
stream that hands out those views): the runner's own methods run unchanged.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

OUT = Path(__file__).resolve().parent / "flux_blocks_tiny.safetensors"
OUT_RUNNER = Path(__file__).resolve().parent / "flux_runner_tiny.safetensors"

# A small FLUX-shaped config: hidden 32, 2 heads of 16 (RoPE axes 4+6+6), mlp 64.
HIDDEN, HEADS, MLP, AXES = 32, 2, 64, (4, 6, 6)
BATCH, LT, GRID = 2, 8, 4  # 8 text tokens, 4x4 image tokens


class DenseView:
    """Minimal stand-in for selas.store.UnitView over plain fp32 tensors, decoded to ``dtype``
    (the compute dtype) as UnitView.get does (store.py:265-293)."""

    def __init__(self, tensors, dtype=torch.float32):
        self.t = tensors
        self.dtype = dtype

    def has(self, name):
        return name in self.t

    def get(self, name, dtype=None):
        return self.t[name].to(dtype or self.dtype)

    def linear(self, x, prefix, dtype=None):
        """F.linear(x, W, b) in the compute dtype. In bf16 it is evaluated as the GPU BLAS call of the
        reference evaluates it: operands in bf16, fp32 accumulation and bias, one rounding (torch's CPU
        bf16 matmul rounds differently on strided inputs such as the attention slices)."""
        dt = dtype or self.dtype
        b = self.t.get(prefix + ".bias")
        w = self.t[prefix + ".weight"].to(dt)
        if dt == torch.float32:
            return torch.nn.functional.linear(x, w, b)
        y = torch.nn.functional.linear(x.to(dt).float(), w.float(), None if b is None else b.to(dt).float())
        return y.to(dt)


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

    f32, bf16 = torch.float32, torch.bfloat16
    with torch.no_grad():
        img_o, txt_o = double_block(DenseView(dbl), img, txt, dmod, cos, sin, cfg, f32, False, EAGER)
        x = torch.cat((txt, img), dim=1)
        x_o = single_block(DenseView(sgl), x, smod, cos, sin, cfg, f32, False, EAGER)
        x_g = single_block(DenseView(sgl), x * 3e4, smod, cos, sin, cfg, f32, True, EAGER)
        fin = final_layer(DenseView(glb), img, fmod, f32, EAGER)
        # The same blocks in the bf16 compute dtype (weights decoded to bf16, fp32 residual streams).
        img_b, txt_b = double_block(DenseView(dbl, bf16), img, txt, dmod.to(bf16), cos, sin, cfg, bf16, False, EAGER)
        x_b = single_block(DenseView(sgl, bf16), x, smod.to(bf16), cos, sin, cfg, bf16, False, EAGER)
        fin_b = final_layer(DenseView(glb, bf16), img, fmod.to(bf16), bf16, EAGER)

    tensors = {"in.img": img, "in.txt": txt, "in.dmod": dmod, "in.smod": smod, "in.fmod": fmod, "in.ids": ids,
               "out.cos": cos, "out.sin": sin, "out.double.img": img_o, "out.double.txt": txt_o,
               "out.single.x": x_o, "out.single_guard.x": x_g, "out.final": fin,
               "out.bf16.double.img": img_b, "out.bf16.double.txt": txt_b, "out.bf16.single.x": x_b,
               "out.bf16.final": fin_b}
    tensors.update({f"w.double.{k}": v for k, v in dbl.items()})
    tensors.update({f"w.single.{k}": v for k, v in sgl.items()})
    tensors.update({f"w.globals.{k}": v for k, v in glb.items()})
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(OUT),
              metadata={"hidden": str(HIDDEN), "heads": str(HEADS), "mlp": str(MLP), "axes": ",".join(map(str, AXES)),
                        "batch": str(BATCH), "lt": str(LT), "grid": str(GRID)})
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


# The runner golden: a two-double, two-single-block model, 3 steps, batch 2.
R_DOUBLE, R_SINGLE, R_CTX, R_VEC, R_STEPS = 2, 2, 24, 16, 3


class _Stream:
    """Hands out the views of named units (the acquire/release interface of selas's weight streams)."""

    def __init__(self, views):
        self.views = views

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False

    def acquire(self, name):
        return self.views[name]

    def release(self, name):
        pass


class _Store:
    def __init__(self, views):
        self.views = views
        self.device = torch.device("cpu")
        self.profile = False

    def stream(self, names, cyclic=False):
        return _Stream(self.views)


def runner(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from selas.models.flux import EAGER, FluxConfig, FluxRunner, double_names, main_order, mod_order, single_names
    from selas.sampling import get_schedule, image_ids, text_ids

    cfg = FluxConfig(hidden=HIDDEN, heads=HEADS, mlp_hidden=MLP, depth_double=R_DOUBLE, depth_single=R_SINGLE,
                     in_channels=64, context_dim=R_CTX, vec_dim=R_VEC, axes_dim=AXES, guidance_embed=True)
    g = torch.Generator().manual_seed(4321)
    d, m = HIDDEN, MLP
    units: dict[str, dict] = {"globals": {}}
    glb = units["globals"]
    for name, i, o in (("img_in", 64, d), ("txt_in", R_CTX, d), ("time_in.in_layer", 256, d),
                       ("time_in.out_layer", d, d), ("guidance_in.in_layer", 256, d), ("guidance_in.out_layer", d, d),
                       ("vector_in.in_layer", R_VEC, d), ("vector_in.out_layer", d, d),
                       ("final_layer.adaLN_modulation.1", d, 2 * d), ("final_layer.linear", d, 64)):
        _lin(glb, g, name, i, o)
    for name in double_names(cfg):
        u = units.setdefault(name, {})
        mu = units.setdefault(name + ".mod", {})
        for s in ("img", "txt"):
            _lin(u, g, f"{s}_attn.qkv", d, 3 * d)
            _lin(u, g, f"{s}_attn.proj", d, d)
            _lin(u, g, f"{s}_mlp.0", d, m)
            _lin(u, g, f"{s}_mlp.2", m, d)
            for q in ("query", "key"):
                u[f"{s}_attn.norm.{q}_norm.scale"] = 1 + 0.1 * torch.randn(d // HEADS, generator=g)
            _lin(mu, g, f"{s}_mod.lin", d, 6 * d)
    for name in single_names(cfg):
        u = units.setdefault(name, {})
        _lin(u, g, "linear1", d, 3 * d + m)
        _lin(u, g, "linear2", d + m, d)
        for q in ("query", "key"):
            u[f"norm.{q}_norm.scale"] = 1 + 0.1 * torch.randn(d // HEADS, generator=g)
        _lin(units.setdefault(name + ".mod", {}), g, "modulation.lin", d, 3 * d)

    f32 = torch.float32
    views = {n: DenseView(t, f32) for n, t in units.items()}
    r = FluxRunner.__new__(FluxRunner)  # the runner's own methods over stand-in weights
    r.store, r.k, r.cfg, r.dt, r.guard = _Store(views), EAGER, cfg, f32, False
    r.g, r.main, r.doubles, r.singles = views["globals"], main_order(cfg), double_names(cfg), single_names(cfg)
    r.mod_units, r.micro_batch, r._stream = mod_order(cfg), None, _Stream(views)

    li = GRID * GRID
    sigmas = get_schedule(R_STEPS, li)
    guidance = 3.5
    pooled = torch.randn(BATCH, R_VEC, generator=g)
    txt = torch.randn(BATCH, LT, R_CTX, generator=g)
    lat = torch.randn(BATCH, li, 64, generator=g)
    img_ids, txt_ids = image_ids(16 * GRID, 16 * GRID), text_ids(LT)
    out = {"in.sigmas": torch.tensor(sigmas, dtype=torch.float64), "in.guidance": torch.tensor([guidance]),
           "in.pooled": pooled, "in.txt": txt, "in.latents": lat, "in.img_ids": img_ids, "in.txt_ids": txt_ids}
    with torch.no_grad():
        from selas.models.flux import mlp_embed, timestep_embedding

        t = torch.tensor(list(sigmas[:-1]), dtype=torch.float32)
        out["out.temb"] = timestep_embedding(t, 256)
        out["out.time_mlp"] = mlp_embed(views["globals"], "time_in", out["out.temb"])
        svecs = [r.svec(sigmas, guidance, pooled[i:i + 1]) for i in range(BATCH)]
        per_image = r.modulations(svecs)
        mods = {n: torch.cat([pm[n] for pm in per_image], dim=1) for n in r.main}
        cond = r.prepare(sigmas, guidance, pooled, txt, img_ids, txt_ids, mods=mods)
        x = lat
        for s in range(2):
            pred, _ = r.step(s, x, cond)
            out[f"out.step{s}.pred"] = pred
            x = x + (sigmas[s + 1] - sigmas[s]) * pred
            out[f"out.step{s}.x"] = x
    for i, sv in enumerate(svecs):
        out[f"out.svec{i}"] = sv
    for n, t_ in mods.items():
        out[f"out.mods.{n}"] = t_
    out.update({"out.final_mod": cond.final_mod, "out.txt": cond.txt, "out.cos": cond.cos, "out.sin": cond.sin})
    for n, t_ in units.items():
        out.update({f"w.{n}.{k}": v for k, v in t_.items()})
    save_file({k: v.contiguous() for k, v in out.items()}, str(OUT_RUNNER),
              metadata={"hidden": str(HIDDEN), "heads": str(HEADS), "mlp": str(MLP), "axes": ",".join(map(str, AXES)),
                        "batch": str(BATCH), "lt": str(LT), "grid": str(GRID), "double": str(R_DOUBLE),
                        "single": str(R_SINGLE), "context": str(R_CTX), "vec": str(R_VEC), "steps": str(R_STEPS)})
    print(f"wrote {OUT_RUNNER} ({OUT_RUNNER.stat().st_size} bytes)")


if __name__ == "__main__":
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    main(root)
    runner(root)
