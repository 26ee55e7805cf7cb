"""Oracle of the FLUX block composition (torch on the CPU): test infrastructure only.

Restates selas/models/flux.py: FluxConfig 44-73, _attention 135-138,
mlp_embed 150-151, double_block 300-324, single_block 327-338,
final_layer 341-343, unit_flops 349-360, FluxRunner.svec 411-425 and the
body of FluxRunner.step 527-582 without the step cache, plus the Euler update
of selas/pipeline.py:489. Blocks take any ``w`` with ``.get``/``.linear`` and
any ``k`` with the seven segment methods, exactly as the reference's do.

``OracleUnit`` is the checker's weight view: NF4 tensors are decoded with the
reference decode (oracle.nf4) to the exact operand the reference multiplies
with, and linears run in fp32 on the CPU.

Pinned by golden vectors written with the reference's own functions
(tests/golden/make_golden.py; tests/test_oracle_flux.py).
"""

from __future__ import annotations

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
                vals = onf4.decode(np.asarray(parts["packed"]), np.asarray(parts["absmax"]), int(meta["blocksize"]),
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
        dt = dtype or self.dtype
        w = self.t[prefix + ".weight"].to(dt)
        b = self.t.get(prefix + ".bias")
        return F.linear(x.to(dt), w, None if b is None else b.to(dt))


def attention(q, k, v):
    """Scaled dot-product attention over [B, H, L, Dh] -> [B, L, H*Dh] (flux.py:135-138), in fp32."""
    b, h, l, d = q.shape
    out = F.scaled_dot_product_attention(q.float(), k.float(), v.float()).to(q.dtype)
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
