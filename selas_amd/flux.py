"""FLUX.1 blocks and step on the gfx950 kernels: the callers of the NF4 hot path.

The block functions follow selas/models/flux.py (double_block 300-324,
single_block 327-338, final_layer 341-343) with ``w.linear`` going to the fused
NF4 linear and ``k`` defaulting to the fused segment kernels. Attention is the
fused gfx950 kernel (selas_amd.attention) in place of the reference's SDPA call
(flux.py:135-138), with SDPA for the shapes the kernel does not take.

``RandomFlux`` builds a FLUX-shaped model with random weights NF4-encoded on
the GPU (the reference's convert step quantizes every 2-D block weight, keeps
norm scales in fp32, biases and the ``globals`` unit raw: convert.py:144-187).
``FluxRunner`` drives it as the reference's runner does: svec (flux.py:411-425),
the hoisted modulations (428-445), prepare (448-465), step (527-582, without
the step cache) and the sampler loop's Euler update with its finiteness check
(selas/pipeline.py:483-494).
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
    """[B, H, L, Dh] -> [B, L, H*Dh]: the fused gfx950 kernel (selas_amd.attention, any L), or SDPA for
    the shapes it does not take (head dim other than 128, dtypes other than bf16). ``out``: optional
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


# RandomFlux.step runs each block's closing residual add together with the next block's mod_in
# (gated_add_mod) when the two blocks are of one kind.
CHAIN_BLOCKS = True


def _fp32_vectors(vs: list[torch.Tensor]) -> list[torch.Tensor]:
    """[B, n_i] vectors as fp32 views of one converted [B, sum n_i] tensor (a copy and one conversion
    for all of them); vectors already fp32 are returned as they are."""
    if all(v.dtype == torch.float32 for v in vs):
        return vs
    flat = torch.cat([v.reshape(v.shape[0], -1) for v in vs], dim=-1).float()
    return list(flat.split([v.shape[-1] for v in vs], dim=-1))


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


def double_block(w, img, txt, mod, cos, sin, cfg: FluxConfig, dt, guard: bool, k: Kernels = FUSED, h=None,
                 next_mod=None):
    """img [B, Li, D] fp32, txt [B, Lt, D] fp32, mod [B, 12D] (img 6D | txt 6D).

    ``h``: the (img, txt) inputs of the attention linears, mod_in of img and txt with this block's first
    shift and scale, when the previous block computed them. With ``next_mod`` (the next double block's
    [B, 12D]) the closing residual adds also compute the next block's ``h`` in the same pass
    (gated_add_mod) and the result is ``(img, txt, h_next)``."""
    m = mod.float().unsqueeze(1).chunk(12, dim=-1)
    i_sh1, i_sc1, i_g1, i_sh2, i_sc2, i_g2 = m[:6]
    t_sh1, t_sc1, t_g1, t_sh2, t_sc2, t_g2 = m[6:]
    lt = txt.shape[1]
    f32 = torch.float32
    if h is None:
        h = (k.mod_in(img, i_sh1, i_sc1, dt), k.mod_in(txt, t_sh1, t_sc1, dt))
    iqkv, tqkv = _linear_pair(w, (h[0], "img_attn.qkv"), (h[1], "txt_attn.qkv"))
    del h
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
    if next_mod is not None:
        n = next_mod.float().unsqueeze(1).chunk(12, dim=-1)
        img, hi = k.gated_add_mod(img, i_g2, oi, n[0], n[1], dt, guard)
        txt, ht = k.gated_add_mod(txt, t_g2, ot, n[6], n[7], dt, guard)
        return img, txt, (hi, ht)
    img = k.gated_add(img, i_g2, oi, guard)
    txt = k.gated_add(txt, t_g2, ot, guard)
    return img, txt


def single_block(w, x, mod, cos, sin, cfg: FluxConfig, dt, guard: bool, k: Kernels = FUSED, h=None,
                 next_mod=None):
    """x [B, Lt+Li, D] fp32, mod [B, 3D].

    ``h``: linear1's input, mod_in(x) with this block's shift and scale, when the previous block computed
    it. With ``next_mod`` (the next single block's [B, 3D]) the closing residual add also computes the next
    block's ``h`` in the same pass (gated_add_mod) and the result is ``(x, h_next)``."""
    sh, sc, g = mod.float().unsqueeze(1).chunk(3, dim=-1)
    f32 = torch.float32
    if h is None:
        h = k.mod_in(x, sh, sc, dt)

    def close(out):
        if next_mod is None:
            return k.gated_add(x, g, out, guard)
        nsh, nsc, _ = next_mod.float().unsqueeze(1).chunk(3, dim=-1)
        return k.gated_add_mod(x, g, out, nsh, nsc, dt, guard)

    if _fused_gelu(w, k):
        # linear1 writes its MLP columns, GELU'd, straight into linear2's input [attention | GELU(mlp)] and
        # the attention its output into the first columns: the bits of k.attn_mlp without its round trip.
        b, l, d = x.shape
        cat = torch.empty(b, l, d + cfg.mlp_hidden, dtype=dt, device=x.device)
        ((qkv, _),) = w.linear_gelu_many([(h, "linear1", cfg.mlp_hidden, cat[..., d:])])
        del h
        q, kk, v = k.qkv_single(qkv, w.get("norm.query_norm.scale", f32), w.get("norm.key_norm.scale", f32), cos,
                                sin, cfg.heads, dt)
        del qkv
        attention(q, kk, v, out=cat[..., :d])
        del q, kk, v
        out = w.linear(cat, "linear2")
        del cat
        return close(out)
    h = w.linear(h, "linear1")
    qkv, mlp = h.split([3 * cfg.hidden, cfg.mlp_hidden], dim=-1)
    q, kk, v = k.qkv_single(qkv, w.get("norm.query_norm.scale", f32), w.get("norm.key_norm.scale", f32), cos, sin,
                            cfg.heads, dt)
    a = attention(q, kk, v)
    del q, kk, v, qkv
    out = w.linear(k.attn_mlp(a, mlp), "linear2")
    del h, mlp, a
    return close(out)


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
    def step(self, latents, txt, mods_s, final_mod_s, cos, sin, k: Kernels = FUSED,
             micro_batch: int | None = None) -> torch.Tensor:
        """Velocity for one step (flux.py:527-582). latents [B, Li, 64] fp32, txt [B, Lt, D] fp32,
        mods_s: per block [B, kD] for this step, final_mod_s [B, 2D]. ``micro_batch``: each block runs
        the batch in chunks of at most that many images, block by block (flux.py:492-524)."""
        cfg, dt, guard = self.cfg, self.dt, self.dt == torch.float16
        # The blocks use their modulation vectors in fp32 (each block converts its own, flux.py:302, 327):
        # one conversion of all of them is exact and saves a small kernel per block.
        *mods_s, final_mod_s = _fp32_vectors([*mods_s, final_mod_s])
        img = self.globals.linear(latents.to(dt), "img_in").float()
        lt = txt.shape[1]
        nd, ns = len(self.doubles), len(self.singles)
        # Between blocks of one kind, the closing residual add and the next block's mod_in run as one
        # pass (gated_add_mod); the bits are those of the two kernels (same fp32 residual, same statistics).
        chain = CHAIN_BLOCKS and isinstance(k, Kernels)
        b = latents.shape[0]
        mb = micro_batch or b
        chunks = [(a, min(b, a + mb)) for a in range(0, b, mb)]
        h = None
        for i, w in enumerate(self.doubles):
            nxt = mods_s[i + 1] if chain and i + 1 < nd else None
            if len(chunks) == 1:
                r = double_block(w, img, txt, mods_s[i], cos, sin, cfg, dt, guard, k, h, nxt)
                img, txt, h = r if nxt is not None else (*r, None)
                continue
            outs = [double_block(w, img[a:e], txt[a:e], mods_s[i][a:e], cos, sin, cfg, dt, guard, k,
                                 None if h is None else (h[0][a:e], h[1][a:e]),
                                 None if nxt is None else nxt[a:e]) for a, e in chunks]
            img, txt = torch.cat([o[0] for o in outs]), torch.cat([o[1] for o in outs])
            h = (torch.cat([o[2][0] for o in outs]), torch.cat([o[2][1] for o in outs])) if nxt is not None else None
            del outs
        x = torch.cat((txt, img), dim=1)
        del txt, img
        h = None
        for j, w in enumerate(self.singles):
            nxt = mods_s[nd + j + 1] if chain and j + 1 < ns else None
            if len(chunks) == 1:
                r = single_block(w, x, mods_s[nd + j], cos, sin, cfg, dt, guard, k, h, nxt)
                x, h = r if nxt is not None else (r, None)
                continue
            outs = [single_block(w, x[a:e], mods_s[nd + j][a:e], cos, sin, cfg, dt, guard, k,
                                 None if h is None else h[a:e], None if nxt is None else nxt[a:e]) for a, e in chunks]
            if nxt is not None:
                x, h = torch.cat([o[0] for o in outs]), torch.cat([o[1] for o in outs])
            else:
                x, h = torch.cat(outs), None
            del outs
        return final_layer(self.globals, x[:, lt:], final_mod_s, dt, k)


# --------------------------------------------------------------------------- runner


def timestep_embedding(t: torch.Tensor, dim: int = 256, max_period: float = 10000.0,
                       time_factor: float = 1000.0) -> torch.Tensor:
    """Sinusoidal embedding [N, dim] fp32 of times t [N] on t's device (flux.py:95-103)."""
    t = time_factor * t.float()
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    args = t[:, None] * freqs[None]
    emb = torch.cat([torch.cos(args), torch.sin(args)], dim=-1)
    if dim % 2:
        emb = torch.cat([emb, torch.zeros_like(emb[:, :1])], dim=-1)
    return emb


def mlp_embed(w, prefix: str, x: torch.Tensor) -> torch.Tensor:
    """in_layer, SiLU, out_layer (flux.py:150-151)."""
    return w.linear(F.silu(w.linear(x, prefix + ".in_layer")), prefix + ".out_layer")


def text_ids(length: int, device=None) -> torch.Tensor:
    """Zero position ids [length, 3] of the text tokens (selas/sampling.py:68-69)."""
    return torch.zeros(length, 3, device=device)


def get_schedule(num_steps: int, image_seq_len: int, base_shift: float = 0.5, max_shift: float = 1.15,
                 shift: bool = True) -> list[float]:
    """num_steps + 1 sigmas from 1 to 0 with FLUX-dev's resolution-dependent shift (selas/sampling.py:10-27)."""
    ts = [1.0 - i / num_steps for i in range(num_steps + 1)]
    if not shift:
        return ts
    x1, x2 = 256.0, 4096.0
    slope = (max_shift - base_shift) / (x2 - x1)
    mu = slope * image_seq_len + (base_shift - slope * x1)

    def shifted(t: float) -> float:
        if t <= 0.0:
            return 0.0
        if t >= 1.0:
            return 1.0
        return math.exp(mu) / (math.exp(mu) + (1.0 / t - 1.0))

    return [shifted(t) for t in ts]


@dataclass
class FluxConditioning:
    """Everything a step needs besides the latents (flux.py:365-373): per block [S, B, kD] modulations,
    the final layer's [S, B, 2D], the text stream after txt_in [B, Lt, D] fp32 and the RoPE tables."""

    sigmas: list
    mods: dict
    final_mod: torch.Tensor
    txt: torch.Tensor
    cos: torch.Tensor
    sin: torch.Tensor
    l_txt: int


@dataclass
class StepInfo:
    """What a step did (flux.py:376-379): every step here runs in full."""

    decision: str = "full"
    distance: float | None = None


class FluxRunner:
    """The reference runner's prologue and step (flux.py:392-582) over a model whose units are resident
    on one GPU (``RandomFlux``): no weight streaming, every modulation linear of an image in one grouped
    launch. Block names follow the reference ("double.i", "single.j"). ``micro_batch`` runs each block
    over the batch in chunks of at most that many images (the reference's block-major micro-batching,
    flux.py:492-524): peak activation memory follows the chunk, and every image gets the bits of the
    unchunked step except in the tiles of a tiled linear that the batch's size makes it split over K."""

    def __init__(self, model: RandomFlux, kernels: Kernels = FUSED, micro_batch: int | None = None):
        if micro_batch is not None and micro_batch < 1:
            raise ValueError(f"micro_batch must be a positive image count, got {micro_batch}")
        self.model = model
        self.k = kernels
        self.micro_batch = micro_batch
        self.cfg = model.cfg
        self.dt = model.dt
        self.guard = model.dt == torch.float16
        self.g = model.globals
        self.doubles = [f"double.{i}" for i in range(len(model.doubles))]
        self.singles = [f"single.{i}" for i in range(len(model.singles))]
        self.main = self.doubles + self.singles

    @torch.no_grad()
    def svec(self, sigmas, guidance: float, pooled: torch.Tensor) -> torch.Tensor:
        """silu(vec) [S, 1, D] for one image (``pooled`` [1, vec_dim]): timestep + guidance + pooled-text
        embeddings (flux.py:411-425)."""
        cfg, g, dt, dev = self.cfg, self.g, self.dt, self.model.device
        t = torch.tensor(list(sigmas[:-1]), dtype=torch.float32, device=dev)
        vec = mlp_embed(g, "time_in", timestep_embedding(t, 256).to(dt)).float()[:, None, :]
        if cfg.guidance_embed:
            gv = torch.full((1,), float(guidance), dtype=torch.float32, device=dev)
            vec = vec + mlp_embed(g, "guidance_in", timestep_embedding(gv, 256).to(dt)).float()[None]
        vec = vec + mlp_embed(g, "vector_in", pooled.to(dev, dt)).float()[None]
        return F.silu(vec).to(dt)

    @torch.no_grad()
    def modulations(self, svecs: list[torch.Tensor]) -> list[dict[str, torch.Tensor]]:
        """Every block's modulation vectors [S, 1, kD] for each image's svec (flux.py:428-445)."""
        return [dict(zip(self.main, self.model.modulations(sv))) for sv in svecs]

    @torch.no_grad()
    def prepare(self, sigmas, guidance: float, pooled: torch.Tensor, txt: torch.Tensor, img_ids: torch.Tensor,
                txt_ids: torch.Tensor, mods: dict[str, torch.Tensor] | None = None) -> FluxConditioning:
        """Everything that does not depend on the latents, once per batch (flux.py:448-465). ``mods``: the
        batch's modulation vectors {block: [S, B, kD]} when already known."""
        cfg, g, dt, dev = self.cfg, self.g, self.dt, self.model.device
        svecs = [self.svec(sigmas, guidance, pooled[i:i + 1]) for i in range(pooled.shape[0])]
        if mods is None:
            per_image = self.modulations(svecs)
            mods = {n: torch.cat([m[n] for m in per_image], dim=1) for n in self.main}
        final_mod = torch.cat([g.linear(sv, "final_layer.adaLN_modulation.1") for sv in svecs], dim=1)
        txt_h = g.linear(txt.to(dev, dt), "txt_in").float()
        ids = torch.cat((txt_ids, img_ids), dim=0).to(dev)
        cos, sin = rope_tables(ids, cfg.axes_dim, cfg.theta)
        return FluxConditioning(list(sigmas), mods, final_mod, txt_h, cos, sin, txt.shape[1])

    @torch.no_grad()
    def step(self, s: int, latents: torch.Tensor, cond: FluxConditioning, cache=None):
        """Velocity for step ``s`` from packed latents [B, Li, 64] fp32 (flux.py:527-582): (velocity, StepInfo).
        The reference's optional step cache is not part of this path: ``cache`` must be None or inactive."""
        if cache is not None and getattr(cache, "active", False):
            raise NotImplementedError("the step cache is not supported by selas_amd's runner")
        mods_s = [cond.mods[n][s] for n in self.main]
        out = self.model.step(latents, cond.txt, mods_s, cond.final_mod[s], cond.cos, cond.sin, self.k,
                              self.micro_batch)
        return out, StepInfo()

    @torch.no_grad()
    def denoise(self, x: torch.Tensor, cond: FluxConditioning, on_step=None) -> torch.Tensor:
        """The sampler loop (selas/pipeline.py:483-494): per step the velocity, the Euler update
        x + (sigma[s+1] - sigma[s]) * v and a check that the latents stay finite (FloatingPointError
        otherwise). ``on_step(s, steps)`` is called after each step."""
        sig = cond.sigmas
        steps = len(sig) - 1
        for s in range(steps):
            pred, _ = self.step(s, x, cond)
            x = euler_update(x, sig, s, pred, self.dt)
            if on_step is not None:
                on_step(s, steps)
        return x


def euler_update(x: torch.Tensor, sigmas, s: int, pred: torch.Tensor, dt=torch.bfloat16) -> torch.Tensor:
    """x + (sigma[s+1] - sigma[s]) * pred, raising FloatingPointError when the result is not finite
    (selas/pipeline.py:489-494)."""
    x = x + (sigmas[s + 1] - sigmas[s]) * pred
    if not bool(torch.isfinite(x).all()):
        hint = " (fp16 overflow: retry with --dtype fp32)" if dt == torch.float16 else ""
        raise FloatingPointError(f"non-finite latents after step {s + 1}/{len(sigmas) - 1} in {dt}{hint}")
    return x
