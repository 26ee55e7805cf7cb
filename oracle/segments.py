"""Oracle of the FLUX elementwise segments (torch on the CPU): test infrastructure only.

Restates selas/models/flux.py (line numbers there):
  timestep_embedding 95-103, rope_tables 106-114, apply_rope 117-121,
  qk_rms 124-126, _heads 129-132, _res 141-143, _ln 146-147,
  _mod_in 164-166, _gated_add 169-171, _gated_add_mod 174-176,
  _qkv_double 179-185, _qkv_single 188-191, _gelu 194-195, _attn_mlp 198-200.

All arithmetic happens in fp32 (or fp64 where the reference uses fp64), with
the casts to the compute dtype where the reference casts.

Pinned by (tests/test_oracle_segments.py): LayerNorm against torch's
F.layer_norm in fp64 and the zero-mean / unit-variance invariant; RMSNorm's
unit-RMS invariant; RoPE against complex multiplication by exp(i*angle), its
norm preservation and the relative-position property of dot products;
rope_tables' closed-form special cases (position 0, first frequency = angle p);
GELU against F.gelu(approximate="tanh"); the head split by one-hot probes;
the fp16 guard clamp on explicit values.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

FP16_MAX = 65504.0


def timestep_embedding(t: torch.Tensor, dim: int = 256, max_period: float = 10000.0, time_factor: float = 1000.0):
    t = time_factor * t.float()
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32) / half)
    args = t[:, None] * freqs[None]
    emb = torch.cat([torch.cos(args), torch.sin(args)], dim=-1)
    if dim % 2:
        emb = torch.cat([emb, torch.zeros_like(emb[:, :1])], dim=-1)
    return emb


def rope_tables(ids: torch.Tensor, axes_dim, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [L, sum(axes_dim)/2] fp32 from position ids [L, n_axes], angles in fp64."""
    parts = []
    for i, d in enumerate(axes_dim):
        omega = theta ** (-(torch.arange(0, d, 2, dtype=torch.float64) / d))
        parts.append(ids[:, i].double()[:, None] * omega[None])
    ang = torch.cat(parts, dim=-1)
    return ang.cos().float(), ang.sin().float()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotates the interleaved pairs (x[2i], x[2i+1]) of fp32 x [B, H, L, Dh]."""
    a, b = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = a * cos - b * sin
    out[..., 1::2] = a * sin + b * cos
    return out


def qk_rms(x: torch.Tensor, scale: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * scale


def heads(qkv: torch.Tensor, n_heads: int):
    """[B, L, 3*H*Dh] -> q, k, v [B, H, L, Dh]; channel = which*H*Dh + h*Dh + d."""
    b, l, c = qkv.shape
    x = qkv.reshape(b, l, 3, n_heads, c // (3 * n_heads)).permute(2, 0, 3, 1, 4)
    return x[0], x[1], x[2]


def res(y: torch.Tensor, guard: bool) -> torch.Tensor:
    y = y.float()
    return y.clamp(-FP16_MAX, FP16_MAX) if guard else y


def ln(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """LayerNorm over the last dim, no affine: (x - mean) / sqrt(biased var + eps); fp32 (fp64 stays fp64)."""
    x = x if x.dtype == torch.float64 else x.float()
    mean = x.mean(-1, keepdim=True)
    var = (x - mean).pow(2).mean(-1, keepdim=True)
    return (x - mean) / torch.sqrt(var + eps)


def mod_in(x, shift, scale, dt):
    return (ln(x) * (1 + scale) + shift).to(dt)


def gated_add(x, g, y, guard: bool):
    return x + g * res(y, guard)


def gated_add_mod(x, g, y, shift, scale, dt, guard: bool):
    x = gated_add(x, g, y, guard)
    return x, mod_in(x, shift, scale, dt)


def qkv_double(tqkv, iqkv, tqs, tks, iqs, iks, cos, sin, n_heads: int, dt):
    tq, tk, tv = heads(tqkv, n_heads)
    iq, ik, iv = heads(iqkv, n_heads)
    q = apply_rope(torch.cat((qk_rms(tq, tqs), qk_rms(iq, iqs)), dim=2), cos, sin).to(dt)
    k = apply_rope(torch.cat((qk_rms(tk, tks), qk_rms(ik, iks)), dim=2), cos, sin).to(dt)
    return q, k, torch.cat((tv, iv), dim=2)


def qkv_single(qkv, qs, ks, cos, sin, n_heads: int, dt):
    q, k, v = heads(qkv, n_heads)
    return apply_rope(qk_rms(q, qs), cos, sin).to(dt), apply_rope(qk_rms(k, ks), cos, sin).to(dt), v.contiguous()


def gelu(h: torch.Tensor) -> torch.Tensor:
    """GELU, tanh approximation, evaluated in fp32 and cast back to h's dtype."""
    x = h.float()
    y = 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x * x * x)))
    return y.to(h.dtype)


def attn_mlp(attn, mlp):
    return torch.cat((attn, gelu(mlp)), dim=2)


class OracleKernels:
    """The segments above under the names of selas.models.flux.Kernels (flux.py:206-212)."""

    compiled = False
    mod_in = staticmethod(mod_in)
    gated_add = staticmethod(gated_add)
    gated_add_mod = staticmethod(gated_add_mod)
    qkv_double = staticmethod(qkv_double)
    qkv_single = staticmethod(qkv_single)
    gelu = staticmethod(gelu)
    attn_mlp = staticmethod(attn_mlp)


def layer_norm_library(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """torch's own LayerNorm (a library routine), used to pin ``ln``."""
    return F.layer_norm(x, (x.shape[-1],), eps=eps)
