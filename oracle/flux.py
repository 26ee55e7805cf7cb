"""Oracle of the FLUX block composition (torch on the CPU): test infrastructure only.

Restates selas/models/flux.py: FluxConfig 44-73, _attention 135-138,
mlp_embed 150-151, double_block 300-324, single_block 327-338,
final_layer 341-343, unit_flops 349-360, FluxRunner.svec 411-425,
FluxRunner.modulations 428-445, FluxRunner.prepare 448-465 and the body of
FluxRunner.step 527-582 without the step cache, plus the Euler update and the
finiteness check of selas/pipeline.py:489-494. Blocks take any ``w`` with
``.get``/``.linear`` and any ``k`` with the seven segment methods, exactly as
the reference's do.

``OracleUnit`` is the checker's weight view: NF4 tensors are decoded with the
reference decode (oracle.nf4) to the exact operand the reference multiplies
with. Its linears take the operands in the compute dtype and accumulate in
fp32 with one rounding of the output to the compute dtype, which is the
arithmetic of the GPU BLAS call the reference makes (F.linear in bf16); in
fp32 they are plain fp32 linears.

Pinned by golden vectors written with the reference's own functions
(tests/golden/make_golden.py; tests/test_oracle_flux.py): the blocks in fp32
and in bf16, rope_tables, timestep_embedding, mlp_embed, svec, modulations,
prepare, two steps with their Euler updates; unit_flops against the totals
the reference publishes (docs/PLAN.md:51-52).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import int8_row as oi8
from . import nf4 as onf4
from .segments import OracleKernels, timestep_embedding


@dataclass
class FluxConfig:
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


TINY_FLUX = FluxConfig(hidden=64, heads=4, mlp_hidden=256, depth_double=2, depth_single=3, in_channels=64,
                       context_dim=32, vec_dim=24, axes_dim=(4, 6, 6), guidance_embed=True)


class OracleUnit:
    """Weights of one unit for the oracle: name -> fp32 CPU tensor (NF4 decoded to its operand values)."""

    def __init__(self, tensors: dict[str, torch.Tensor], dtype: torch.dtype = torch.float32):
        self.t = tensors
        self.dtype = dtype

    @classmethod
    def from_encoded(cls, enc: dict, dtype: torch.dtype, operand_dtype: torch.dtype = torch.bfloat16):
        """From {name: (codec, shape, meta, parts)} with CPU numpy/torch parts.

        NF4 and int8_row weights decode to ``operand_dtype`` (the compute dtype the
        reference decodes into) and are held as fp32 values of those bits.
        """
        out = {}
        for name, (codec, shape, meta, parts) in enc.items():
            if codec == "nf4":
                dec = onf4.c_decode if onf4.c_lib() else onf4.decode
                vals = dec(np.asarray(parts["packed"]), np.asarray(parts["absmax"]), int(meta["blocksize"]),
                           meta["code"], onf4.F32)
                w = torch.from_numpy(vals).view(*shape).to(operand_dtype).float()
            elif codec == "int8_row":
                out_code = {torch.bfloat16: oi8.BF16, torch.float16: oi8.F16, torch.float32: oi8.F32}[operand_dtype]
                vals = oi8.decode(np.asarray(parts["q"]), np.asarray(parts["scale"]), out_code)
                if out_code == oi8.BF16:
                    vals = onf4.bf16_to_f32(vals)
                elif out_code == oi8.F16:
                    vals = vals.view(np.float16).astype(np.float32)
                w = torch.from_numpy(np.ascontiguousarray(vals)).view(*shape).float()
            else:
                w = torch.as_tensor(parts["data"]).float()
            out[name] = w
        return cls(out, dtype)

    def has(self, name):
        return name in self.t

    def get(self, name, dtype=None):
        return self.t[name].to(dtype or self.dtype)

    def linear(self, x, prefix, dtype=None):
        """F.linear in the compute dtype: operands rounded to it, fp32 accumulation, bias added in fp32,
        one rounding of the result (fp32 compute dtype: a plain fp32 linear)."""
        dt = dtype or self.dtype
        w = self.t[prefix + ".weight"].to(dt).float()
        b = self.t.get(prefix + ".bias")
        y = F.linear(x.to(dt).float(), w, None if b is None else b.to(dt).float())
        return y.to(dt)


def attention(q, k, v):
    """Scaled dot-product attention over [B, H, L, Dh] -> [B, L, H*Dh] (flux.py:135-138).

    fp32 inputs: fp32 SDPA. bf16 / fp16 inputs: the arithmetic of torch's flash backends, which the
    reference's SDPA call runs on a GPU in those dtypes: fp32 scores and softmax, the probabilities
    exp(s - rowmax) rounded to the compute dtype for the product with v, fp32 row sums of the
    unrounded probabilities, fp32 accumulation and one rounding of the output. (A flash kernel
    subtracts a running maximum tile by tile; with the final maximum the roundings differ only
    where that maximum moved.)"""
    b, h, l, d = q.shape
    if q.dtype == torch.float32:
        out = F.scaled_dot_product_attention(q, k.float(), v.float())
    else:
        out = torch.empty_like(q)
        for i in range(b):  # one [L, L] score matrix at a time
            for j in range(h):
                s = (q[i, j].float() @ k[i, j].float().t()) / math.sqrt(d)
                p = torch.exp(s - s.amax(-1, keepdim=True))
                out[i, j] = ((p.to(q.dtype).float() @ v[i, j].float()) / p.sum(-1, keepdim=True)).to(q.dtype)
    return out.transpose(1, 2).reshape(b, l, h * d)


def mlp_embed(w, prefix, x):
    return w.linear(F.silu(w.linear(x, prefix + ".in_layer")), prefix + ".out_layer")


def double_block(w, img, txt, mod, cos, sin, cfg: FluxConfig, dt, guard: bool, k=OracleKernels, attn=attention):
    m = mod.float().unsqueeze(1).chunk(12, dim=-1)
    i_sh1, i_sc1, i_g1, i_sh2, i_sc2, i_g2 = m[:6]
    t_sh1, t_sc1, t_g1, t_sh2, t_sc2, t_g2 = m[6:]
    lt = txt.shape[1]
    f32 = torch.float32
    iqkv = w.linear(k.mod_in(img, i_sh1, i_sc1, dt), "img_attn.qkv")
    tqkv = w.linear(k.mod_in(txt, t_sh1, t_sc1, dt), "txt_attn.qkv")
    q, kk, v = k.qkv_double(tqkv, iqkv, w.get("txt_attn.norm.query_norm.scale", f32),
                            w.get("txt_attn.norm.key_norm.scale", f32), w.get("img_attn.norm.query_norm.scale", f32),
                            w.get("img_attn.norm.key_norm.scale", f32), cos, sin, cfg.heads, dt)
    a = attn(q, kk, v)
    t_attn, i_attn = a[:, :lt], a[:, lt:]
    img, h = k.gated_add_mod(img, i_g1, w.linear(i_attn, "img_attn.proj"), i_sh2, i_sc2, dt, guard)
    h = w.linear(h, "img_mlp.0")
    img = k.gated_add(img, i_g2, w.linear(k.gelu(h), "img_mlp.2"), guard)
    txt, h = k.gated_add_mod(txt, t_g1, w.linear(t_attn, "txt_attn.proj"), t_sh2, t_sc2, dt, guard)
    h = w.linear(h, "txt_mlp.0")
    txt = k.gated_add(txt, t_g2, w.linear(k.gelu(h), "txt_mlp.2"), guard)
    return img, txt


def single_block(w, x, mod, cos, sin, cfg: FluxConfig, dt, guard: bool, k=OracleKernels, attn=attention):
    sh, sc, g = mod.float().unsqueeze(1).chunk(3, dim=-1)
    f32 = torch.float32
    h = w.linear(k.mod_in(x, sh, sc, dt), "linear1")
    qkv, mlp = h.split([3 * cfg.hidden, cfg.mlp_hidden], dim=-1)
    q, kk, v = k.qkv_single(qkv, w.get("norm.query_norm.scale", f32), w.get("norm.key_norm.scale", f32), cos, sin,
                            cfg.heads, dt)
    a = attn(q, kk, v)
    out = w.linear(k.attn_mlp(a, mlp), "linear2")
    return k.gated_add(x, g, out, guard)


def final_layer(w, img, fmod, dt, k=OracleKernels):
    sh, sc = fmod.float().unsqueeze(1).chunk(2, dim=-1)
    return w.linear(k.mod_in(img, sh, sc, dt), "final_layer.linear").float()


def unit_flops(kind: str, cfg: FluxConfig, l_img: int, l_txt: int, batch: int) -> tuple[float, float]:
    """(linear FLOPs, attention FLOPs) of one unit for one step (flux.py:349-360)."""
    d, m = cfg.hidden, cfg.mlp_hidden
    seq = l_img + l_txt
    attn = 4.0 * batch * seq * seq * d
    if kind == "double":
        return 2.0 * batch * seq * (d * 3 * d + d * d + d * m + m * d), attn
    if kind == "single":
        return 2.0 * batch * seq * (d * (3 * d + m) + (d + m) * d), attn
    return 0.0, 0.0


def svec(g, cfg: FluxConfig, sigmas, guidance: float, pooled: torch.Tensor, dt) -> torch.Tensor:
    """silu(vec) [S, 1, D] for one image (flux.py:411-425)."""
    t = torch.tensor(list(sigmas[:-1]), dtype=torch.float32)
    vec = mlp_embed(g, "time_in", timestep_embedding(t, 256).to(dt)).float()[:, None, :]
    if cfg.guidance_embed:
        gv = torch.full((1,), float(guidance), dtype=torch.float32)
        vec = vec + mlp_embed(g, "guidance_in", timestep_embedding(gv, 256).to(dt)).float()[None]
    vec = vec + mlp_embed(g, "vector_in", pooled.to(dt)).float()[None]
    return F.silu(vec).to(dt)


def modulations(mod_units, svecs, n_double: int):
    """Every block's modulation vectors [S, 1, kD] per image (flux.py:428-445): double blocks concatenate
    the image and text linears, single blocks have one; ``mod_units`` in block order."""
    outs = []
    for sv in svecs:
        per = []
        for i, w in enumerate(mod_units):
            if i < n_double:
                per.append(torch.cat((w.linear(sv, "img_mod.lin"), w.linear(sv, "txt_mod.lin")), dim=-1))
            else:
                per.append(w.linear(sv, "modulation.lin"))
        outs.append(per)
    return outs


@dataclass
class Conditioning:
    """FluxConditioning (flux.py:365-373) for the oracle."""

    sigmas: list
    mods: list  # per block [S, B, kD]
    final_mod: torch.Tensor  # [S, B, 2D]
    txt: torch.Tensor  # [B, Lt, D] fp32
    cos: torch.Tensor
    sin: torch.Tensor
    l_txt: int


def prepare(g, cfg: FluxConfig, sigmas, guidance: float, pooled, txt, img_ids, txt_ids, mods, dt) -> Conditioning:
    """FluxRunner.prepare (flux.py:448-465) with the batch's modulations given ([S, B, kD] per block)."""
    from .segments import rope_tables

    svecs = [svec(g, cfg, sigmas, guidance, pooled[i:i + 1], dt) for i in range(pooled.shape[0])]
    final_mod = torch.cat([g.linear(sv, "final_layer.adaLN_modulation.1") for sv in svecs], dim=1)
    txt_h = g.linear(txt.to(dt), "txt_in").float()
    ids = torch.cat((txt_ids, img_ids), dim=0)
    cos, sin = rope_tables(ids, cfg.axes_dim, cfg.theta)
    return Conditioning(list(sigmas), mods, final_mod, txt_h, cos, sin, txt.shape[1])


def step(g, doubles, singles, cfg: FluxConfig, s: int, latents, cond: Conditioning, dt, k=OracleKernels,
         attn=attention):
    """Velocity for step ``s`` (FluxRunner.step, flux.py:527-582, without the step cache)."""
    guard = dt == torch.float16
    img = g.linear(latents.to(dt), "img_in").float()
    txt = cond.txt
    nd = len(doubles)
    for i, w in enumerate(doubles):
        img, txt = double_block(w, img, txt, cond.mods[i][s], cond.cos, cond.sin, cfg, dt, guard, k, attn)
    x = torch.cat((txt, img), dim=1)
    for j, w in enumerate(singles):
        x = single_block(w, x, cond.mods[nd + j][s], cond.cos, cond.sin, cfg, dt, guard, k, attn)
    return final_layer(g, x[:, cond.l_txt:], cond.final_mod[s], dt, k)


def euler(x, sigmas, s: int, pred):
    """One sampler update x + (sigma[s+1] - sigma[s]) * v, then the finiteness check that raises
    FloatingPointError on non-finite latents (selas/pipeline.py:489-494)."""
    x = x + (sigmas[s + 1] - sigmas[s]) * pred
    if not bool(torch.isfinite(x).all()):
        raise FloatingPointError(f"non-finite latents after step {s + 1}/{len(sigmas) - 1}")
    return x
