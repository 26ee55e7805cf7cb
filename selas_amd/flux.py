"""FLUX.1 blocks and step on the gfx950 kernels: the callers of the NF4 hot path.

The block functions follow selas/models/flux.py (double_block 300-324,
single_block 327-338, final_layer 341-343, FluxRunner.step 527-582 without the
step cache, modulation hoisting 411-445) with ``w.linear`` going to the fused
NF4 linear and ``k`` defaulting to the fused segment kernels. Attention is the
library SDPA call the reference makes (flux.py:135-138), restricted to the
fused flash / memory-efficient backends.

``RandomFlux`` builds a FLUX-shaped model with random weights NF4-encoded on
the GPU (the reference's convert step quantizes every 2-D block weight, keeps
norm scales in fp32, biases and the ``globals`` unit raw: convert.py:144-187).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .codecs import EncodedTensor, encode_int8_row, encode_nf4, encode_raw
from .kernels import FUSED, Kernels
from .linear import UnitView, int8_row_linear_grouped, nf4_linear_grouped


@dataclass
class FluxConfig:
    """selas.models.flux.FluxConfig (flux.py:44-73)."""

    hidden: int = 3072
    heads: int = 24
    mlp_hidden: int = 12288
    depth_double: int = 19
    depth_single: int = 38
    in_channels: int = 64
    context_dim: int = 4096
    vec_dim: int = 768
    axes_dim: tuple = (16, 56, 56)
    theta: float = 10000.0
    guidance_embed: bool = True

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


def rope_tables(ids: torch.Tensor, axes_dim, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [L, head_dim/2] fp32 for position ids [L, n_axes], angles in fp64 (flux.py:106-114)."""
    parts = []
    for i, d in enumerate(axes_dim):
        omega = theta ** (-(torch.arange(0, d, 2, dtype=torch.float64, device=ids.device) / d))
        parts.append(ids[:, i].double()[:, None] * omega[None])
    ang = torch.cat(parts, dim=-1)
    return ang.cos().float(), ang.sin().float()


def image_ids(h: int, w: int, device=None) -> torch.Tensor:
    """(0, row, col) ids of an h x w packed latent grid (selas/sampling.py:58-65)."""
    ids = torch.zeros(h, w, 3, device=device)
    ids[..., 1] = torch.arange(h, device=device)[:, None]
    ids[..., 2] = torch.arange(w, device=device)[None, :]
    return ids.reshape(h * w, 3)


def sdpa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """The reference's attention (flux.py:135-138): SDPA over [B, H, L, Dh] -> [B, L, H*Dh], on torch's
    fused backends only."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    b, h, l, d = q.shape
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        out = F.scaled_dot_product_attention(q, k, v)
    return out.transpose(1, 2).reshape(b, l, h * d)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """[B, H, L, Dh] -> [B, L, H*Dh]: the fused gfx950 kernel (selas_amd.attention), or SDPA for the
    shapes it does not take (head dim other than 128, L not a multiple of 128). ``out``: optional
    destination with equally spaced rows (returned)."""
    from . import _lib
    from .attention import attention as fused_attention

    try:
        return fused_attention(q, k, v, out)
    except _lib.Unsupported:
        a = sdpa_attention(q, k, v)
        if out is None:
            return a
        out.copy_(a)
        return out


def _fused_gelu(w, k) -> bool:
    """The GELU after the MLP input linears goes into the GEMM epilogue when the unit can do that and the
    segments are this package's kernels (whose GELU the epilogue reproduces bit for bit)."""
    from .kernels import Kernels

    return isinstance(k, Kernels) and hasattr(w, "linear_gelu_many")


def _linear_pair(w, a, b):
    """w.linear on two independent (x, prefix) inputs; one launch when ``w`` batches linears."""
    many = getattr(w, "linear_many", None)
    if many is None:
        return w.linear(*a), w.linear(*b)
    ya, yb = many([a, b])
    return ya, yb


def double_block(w, img, txt, mod, cos, sin, cfg: FluxConfig, dt, guard: bool, k: Kernels = FUSED):
    """img [B, Li, D] fp32, txt [B, Lt, D] fp32, mod [B, 12D] (img 6D | txt 6D)."""
    m = mod.float().unsqueeze(1).chunk(12, dim=-1)
    i_sh1, i_sc1, i_g1, i_sh2, i_sc2, i_g2 = m[:6]
    t_sh1, t_sc1, t_g1, t_sh2, t_sc2, t_g2 = m[6:]
    lt = txt.shape[1]
    f32 = torch.float32
    iqkv, tqkv = _linear_pair(w, (k.mod_in(img, i_sh1, i_sc1, dt), "img_attn.qkv"),
                              (k.mod_in(txt, t_sh1, t_sc1, dt), "txt_attn.qkv"))
    q, kk, v = k.qkv_double(tqkv, iqkv, w.get("txt_attn.norm.query_norm.scale", f32),
                            w.get("txt_attn.norm.key_norm.scale", f32), w.get("img_attn.norm.query_norm.scale", f32),
                            w.get("img_attn.norm.key_norm.scale", f32), cos, sin, cfg.heads, dt)
    del iqkv, tqkv
    a = attention(q, kk, v)
    del q, kk, v
    t_attn, i_attn = a[:, :lt], a[:, lt:]
    i_proj, t_proj = _linear_pair(w, (i_attn, "img_attn.proj"), (t_attn, "txt_attn.proj"))
    img, hi = k.gated_add_mod(img, i_g1, i_proj, i_sh2, i_sc2, dt, guard)
    txt, ht = k.gated_add_mod(txt, t_g1, t_proj, t_sh2, t_sc2, dt, guard)
    del i_proj, t_proj
    if _fused_gelu(w, k):
        # mlp.0 with the GELU in its epilogue: the same bits as k.gelu of its output
        (_, hi), (_, ht) = w.linear_gelu_many([(hi, "img_mlp.0", cfg.mlp_hidden, None),
                                               (ht, "txt_mlp.0", cfg.mlp_hidden, None)])
    else:
        hi, ht = _linear_pair(w, (hi, "img_mlp.0"), (ht, "txt_mlp.0"))
        hi, ht = k.gelu(hi), k.gelu(ht)
    oi, ot = _linear_pair(w, (hi, "img_mlp.2"), (ht, "txt_mlp.2"))
    img = k.gated_add(img, i_g2, oi, guard)
    txt = k.gated_add(txt, t_g2, ot, guard)
    return img, txt


def single_block(w, x, mod, cos, sin, cfg: FluxConfig, dt, guard: bool, k: Kernels = FUSED):
    """x [B, Lt+Li, D] fp32, mod [B, 3D]."""
    sh, sc, g = mod.float().unsqueeze(1).chunk(3, dim=-1)
    f32 = torch.float32
    if _fused_gelu(w, k):
        # linear1 writes its MLP columns, GELU'd, straight into linear2's input [attention | GELU(mlp)] and
        # the attention its output into the first columns: the bits of k.attn_mlp without its round trip.
        b, l, d = x.shape
        cat = torch.empty(b, l, d + cfg.mlp_hidden, dtype=dt, device=x.device)
        ((qkv, _),) = w.linear_gelu_many([(k.mod_in(x, sh, sc, dt), "linear1", cfg.mlp_hidden, cat[..., d:])])
        q, kk, v = k.qkv_single(qkv, w.get("norm.query_norm.scale", f32), w.get("norm.key_norm.scale", f32), cos,
                                sin, cfg.heads, dt)
        del qkv
        attention(q, kk, v, out=cat[..., :d])
        del q, kk, v
        out = w.linear(cat, "linear2")
        del cat
        return k.gated_add(x, g, out, guard)
    h = w.linear(k.mod_in(x, sh, sc, dt), "linear1")
    qkv, mlp = h.split([3 * cfg.hidden, cfg.mlp_hidden], dim=-1)
    q, kk, v = k.qkv_single(qkv, w.get("norm.query_norm.scale", f32), w.get("norm.key_norm.scale", f32), cos, sin,
                            cfg.heads, dt)
    a = attention(q, kk, v)
    del q, kk, v, qkv
    out = w.linear(k.attn_mlp(a, mlp), "linear2")
    del h, mlp, a
    return k.gated_add(x, g, out, guard)


def final_layer(w, img, fmod, dt, k: Kernels = FUSED):
    sh, sc = fmod.float().unsqueeze(1).chunk(2, dim=-1)
    return w.linear(k.mod_in(img, sh, sc, dt), "final_layer.linear").float()


def unit_flops(kind: str, cfg: FluxConfig, l_img: int, l_txt: int, batch: int) -> tuple[float, float]:
    """(linear FLOPs, attention FLOPs) of one block for one step (flux.py:349-360)."""
    d, m = cfg.hidden, cfg.mlp_hidden
    seq = l_img + l_txt
    attn = 4.0 * batch * seq * seq * d
    if kind == "double":
        return 2.0 * batch * seq * (d * 3 * d + d * d + d * m + m * d), attn
    if kind == "single":
        return 2.0 * batch * seq * (d * (3 * d + m) + (d + m) * d), attn
    return 0.0, 0.0


# --------------------------------------------------------------------------- random-init model


class _Gen:
    """Draws N(0, std) weights from one large random pool at varying offsets (distinct tensors,
    cheap to make): the pool is regenerated every few tensors."""

    def __init__(self, device, seed: int, pool_elems: int):
        self.g = torch.Generator(device=device).manual_seed(seed)
        self.device = device
        self.n = pool_elems
        self.pool = None
        self.uses = 0

    def normal(self, shape, std: float) -> torch.Tensor:
        n = math.prod(shape)
        if self.pool is None or self.uses >= 8 or n > self.n:
            self.n = max(self.n, n)
            self.pool = torch.randn(self.n + 4096, generator=self.g, device=self.device)
            self.uses = 0
        off = int(torch.randint(0, 4096, (1,), generator=self.g, device=self.device).item()) if n < self.n else 0
        self.uses += 1
        return (self.pool[off: off + n] * std).view(*shape)


def _linear_parts(gen: _Gen, name: str, n_in: int, n_out: int, dt, quant, std: float = 0.02):
    """A linear's weight and bias; ``quant``: False (raw in dt), "nf4" or "int8" (int8_row), the choices
    of selas's convert --quant (convert.py:170-187)."""
    out = {}
    w = gen.normal((n_out, n_in), std)
    if quant == "int8":
        out[name + ".weight"] = encode_int8_row(name + ".weight", w)
    elif quant:
        out[name + ".weight"] = encode_nf4(name + ".weight", w)
    else:
        out[name + ".weight"] = encode_raw(name + ".weight", w, dt)
    out[name + ".bias"] = encode_raw(name + ".bias", gen.normal((n_out,), std), dt)
    return out


class RandomFlux:
    """A FLUX-shaped transformer with random weights, quantized blocks resident on one GPU.

    ``quant``: "nf4" (default) or "int8" (int8_row) for the block and modulation linears."""

    def __init__(self, cfg: FluxConfig, device, dtype=torch.bfloat16, seed: int = 0, n_double=None, n_single=None,
                 with_mods: bool = True, quant: str = "nf4"):
        if quant not in ("nf4", "int8"):
            raise ValueError(f"quant must be 'nf4' or 'int8', got {quant!r}")
        self.cfg, self.device, self.dt = cfg, torch.device(device), dtype
        nd = cfg.depth_double if n_double is None else n_double
        ns = cfg.depth_single if n_single is None else n_single
        d, m, hd = cfg.hidden, cfg.mlp_hidden, cfg.head_dim
        gen = _Gen(self.device, seed, (3 * d + m) * d)

        def norms(prefix):
            return {prefix + q: encode_raw(prefix + q, 1 + gen.normal((hd,), 0.02), torch.float32)
                    for q in ("query_norm.scale", "key_norm.scale")}

        g = {}
        for name, i, o in (("img_in", cfg.in_channels, d), ("txt_in", cfg.context_dim, d),
                           ("time_in.in_layer", 256, d), ("time_in.out_layer", d, d),
                           ("vector_in.in_layer", cfg.vec_dim, d), ("vector_in.out_layer", d, d),
                           ("final_layer.linear", d, cfg.in_channels), ("final_layer.adaLN_modulation.1", d, 2 * d)):
            g.update(_linear_parts(gen, name, i, o, dtype, quant=False))
        if cfg.guidance_embed:
            for name, i, o in (("guidance_in.in_layer", 256, d), ("guidance_in.out_layer", d, d)):
                g.update(_linear_parts(gen, name, i, o, dtype, quant=False))
        self.globals = UnitView(g, dtype)
        self.doubles, self.singles, self.mods = [], [], []
        for _ in range(nd):
            t: dict[str, EncodedTensor] = {}
            for s in ("img", "txt"):
                t.update(_linear_parts(gen, f"{s}_attn.qkv", d, 3 * d, dtype, quant))
                t.update(_linear_parts(gen, f"{s}_attn.proj", d, d, dtype, quant))
                t.update(_linear_parts(gen, f"{s}_mlp.0", d, m, dtype, quant))
                t.update(_linear_parts(gen, f"{s}_mlp.2", m, d, dtype, quant))
                t.update(norms(f"{s}_attn.norm."))
            self.doubles.append(UnitView(t, dtype))
            if with_mods:
                mt = {}
                for s in ("img", "txt"):
                    mt.update(_linear_parts(gen, f"{s}_mod.lin", d, 6 * d, dtype, quant))
                self.mods.append(UnitView(mt, dtype))
        for _ in range(ns):
            t = _linear_parts(gen, "linear1", d, 3 * d + m, dtype, quant)
            t.update(_linear_parts(gen, "linear2", d + m, d, dtype, quant))
            t.update(norms("norm."))
            self.singles.append(UnitView(t, dtype))
            if with_mods:
                self.mods.append(UnitView(_linear_parts(gen, "modulation.lin", d, 3 * d, dtype, quant), dtype))
        del gen

    def nf4_bytes(self) -> int:
        units = self.doubles + self.singles + self.mods
        return sum(e.nbytes for u in units for e in u.tensors.values() if e.codec in ("nf4", "int8_row"))

    def mod_prefixes(self) -> list[tuple[UnitView, str]]:
        nd = len(self.doubles)
        out = []
        for i, u in enumerate(self.mods):
            out += [(u, "img_mod.lin"), (u, "txt_mod.lin")] if i < nd else [(u, "modulation.lin")]
        return out

    @torch.no_grad()
    def modulations(self, sv: torch.Tensor, grouped: bool = True) -> list[torch.Tensor]:
        """Every block's modulation vectors [S, 1, kD] from silu(vec) [S, 1, D] (flux.py:428-445).

        ``grouped`` runs all modulation linears in one launch (same bits as one call per linear)."""
        pre = self.mod_prefixes()
        codecs = {u.tensors[p + ".weight"].codec for u, p in pre}
        if grouped and codecs == {"nf4"}:
            ws = []
            for u, p in pre:
                e = u.tensors[p + ".weight"]
                ws.append((e.parts["packed"], e.parts["absmax"], int(e.meta["blocksize"]), e.meta["code"], e.shape,
                           u.get(p + ".bias")))
            ys = nf4_linear_grouped(sv, ws)
        elif grouped and codecs == {"int8_row"}:
            ws = []
            for u, p in pre:
                e = u.tensors[p + ".weight"]
                ws.append((e.parts["q"], e.parts["scale"], e.shape, u.get(p + ".bias")))
            ys = int8_row_linear_grouped(sv, ws)
        else:
            ys = [u.linear(sv, p) for u, p in pre]
        out, i = [], 0
        for j in range(len(self.mods)):
            if j < len(self.doubles):
                out.append(torch.cat((ys[i], ys[i + 1]), dim=-1))
                i += 2
            else:
                out.append(ys[i])
                i += 1
        return out

    @torch.no_grad()
    def step(self, latents, txt, mods_s, final_mod_s, cos, sin, k: Kernels = FUSED) -> torch.Tensor:
        """Velocity for one step (flux.py:527-582). latents [B, Li, 64] fp32, txt [B, Lt, D] fp32,
        mods_s: per block [B, kD] for this step, final_mod_s [B, 2D]."""
        cfg, dt, guard = self.cfg, self.dt, self.dt == torch.float16
        img = self.globals.linear(latents.to(dt), "img_in").float()
        lt = txt.shape[1]
        nd = len(self.doubles)
        for i, w in enumerate(self.doubles):
            img, txt = double_block(w, img, txt, mods_s[i], cos, sin, cfg, dt, guard, k)
        x = torch.cat((txt, img), dim=1)
        del txt, img
        for j, w in enumerate(self.singles):
            x = single_block(w, x, mods_s[nd + j], cos, sin, cfg, dt, guard, k)
        return final_layer(self.globals, x[:, lt:], final_mod_s, dt, k)
