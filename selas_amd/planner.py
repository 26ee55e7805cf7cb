"""Cost accounting for selas's planner with the fused kernels in place.

selas's planner estimates a unit's step time and reserves memory for the
decoded weight temporaries (selas/pipeline.py:151-165 ``_estimate``, 238-245
``_decode_temp_bytes``) from a throughput profile (selas/hw.py:34-43
``HwProfile``, 128-148 ``measure_matmul`` / ``measure_attention``). With the
fused NF4 and int8_row linears a quantized weight is decoded in registers: it
has no decode temporary and no decode time. This module gives the same
quantities with that taken into account, and measures the profile's GPU
figures with the kernels the step actually runs.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from .flux import FluxConfig, unit_flops

# Codecs whose 2-D weights the fused linears consume without decoding.
FUSED_CODECS = ("nf4", "int8_row")


@dataclass
class HwProfile:
    """Throughput figures the planner divides by (selas/hw.py:34-43, same fields and units)."""

    h2d_bw: float = 11e9            # bytes/s pinned host -> device
    disk_bw: float = 2.0e9          # bytes/s
    matmul_flops: float = 1.05e15   # fused NF4 GEMM at the FLUX block shapes (bf16)
    attn_flops: float = 0.9e15      # fused attention, head dim 128
    mem_bw: float = 5.5e12          # the segment kernels' effective device bandwidth
    dequant_bw: float = 3.0e12      # decoded output bytes/s of the decode kernels
    measured: tuple[str, ...] = field(default_factory=tuple)


def fused_linear(codec: str, shape, meta: dict | None, dtype: torch.dtype) -> bool:
    """True when a linear weight of this codec and shape runs through a fused kernel (no decoded
    temporary): a 2-D NF4 (blocksize 64) or int8_row weight with K % 64 == 0, bf16 compute."""
    if codec not in FUSED_CODECS or len(shape) != 2 or dtype != torch.bfloat16 or int(shape[1]) % 64:
        return False
    return codec != "nf4" or int((meta or {}).get("blocksize", 64)) == 64


def _decoded_is_view(ts, dtype: torch.dtype) -> bool:
    stored = getattr(ts, "stored_dtype", None)
    if stored is None and ts.codec == "raw":
        data = getattr(ts, "parts", {}).get("data")
        stored = None if data is None else str(data.dtype).removeprefix("torch.")
    return ts.codec == "raw" and stored is not None and str(dtype).removeprefix("torch.") == stored


def decoded_bytes(ts, dtype: torch.dtype) -> int:
    """Bytes of the temporary a linear weight is decoded into before its GEMM: 0 for a zero-copy
    view and for fused codecs, else numel x element size (selas/pipeline.py:157-164)."""
    if len(ts.shape) != 2 or _decoded_is_view(ts, dtype) or fused_linear(ts.codec, ts.shape, getattr(ts, "meta", {}),
                                                                          dtype):
        return 0
    n = 1
    for s in ts.shape:
        n *= int(s)
    return n * (torch.finfo(dtype).bits // 8)


def decode_temp_bytes(units, dtype: torch.dtype) -> int:
    """The largest decode temporary over all units' tensors (selas/pipeline.py:238-245); ``units`` is an
    iterable of {name: tensor spec} mappings (objects with ``codec``, ``shape`` and ``meta``)."""
    worst = 0
    for tensors in units:
        for ts in tensors.values():
            worst = max(worst, decoded_bytes(ts, dtype))
    return worst


def estimate_seconds(kind: str, cfg: FluxConfig, l_img: int, l_txt: int, batch: int, tensors, hw: HwProfile,
                     dtype: torch.dtype = torch.bfloat16) -> float:
    """Estimated time of one block for one step (selas/pipeline.py:151-165): linear and attention FLOPs
    over the profile's rates, the elementwise traffic model of the reference (100 bytes per activation
    element) over ``mem_bw``, and the decode temporaries that remain over ``dequant_bw``."""
    lin, att = unit_flops(kind, cfg, l_img, l_txt, batch)
    t = lin / hw.matmul_flops + att / hw.attn_flops
    t += batch * (l_img + l_txt) * cfg.hidden * 100 / hw.mem_bw
    dec = sum(decoded_bytes(ts, dtype) for ts in tensors.values())
    return t + dec / hw.dequant_bw


def _timed(fn, device, reps: int) -> float:
    fn()
    torch.cuda.synchronize(device)
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize(device)
    return (time.perf_counter() - t0) / reps


def measure_matmul(device: torch.device, m: int = 4608, n: int = 12288, k: int = 3072, reps: int = 20) -> float:
    """FLOP/s of the fused NF4 GEMM on a FLUX block shape (selas/hw.py:128-137 times torch.mm)."""
    from .codecs import NF4_CODE, encode_nf4
    from .linear import nf4_linear

    g = torch.Generator(device=device).manual_seed(0)
    e = encode_nf4("w", torch.randn(n, k, generator=g, device=device) * 0.02)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    s = _timed(lambda: nf4_linear(x, e.parts["packed"], e.parts["absmax"], 64, NF4_CODE, (n, k)), device, reps)
    return 2.0 * m * n * k / s


def measure_attention(device: torch.device, L: int = 4608, H: int = 24, D: int = 128, reps: int = 5) -> float:
    """FLOP/s of the block attention as ``flux.attention`` runs it (selas/hw.py:140-148 times SDPA)."""
    from .flux import attention

    g = torch.Generator(device=device).manual_seed(1)
    q = torch.randn(1, H, L, D, generator=g, device=device).to(torch.bfloat16)
    s = _timed(lambda: attention(q, q, q), device, reps)
    return 4.0 * L * L * H * D / s


def measure_dequant(device: torch.device, n: int = 12288, k: int = 3072, reps: int = 10) -> float:
    """Decoded output bytes/s of the NF4 decode kernel (bf16 output), for weights that still decode."""
    from .codecs import encode_nf4, nf4_dequant

    g = torch.Generator(device=device).manual_seed(2)
    e = encode_nf4("w", torch.randn(n, k, generator=g, device=device) * 0.02)
    s = _timed(lambda: nf4_dequant(e.parts["packed"], e.parts["absmax"], 64, e.meta["code"], (n, k), torch.bfloat16),
               device, reps)
    return 2.0 * n * k / s


def measure_profile(device: torch.device, prof: HwProfile | None = None) -> HwProfile:
    """A profile with the GPU figures measured on ``device`` (host and disk figures kept)."""
    prof = prof or HwProfile()
    prof.matmul_flops = measure_matmul(device)
    prof.attn_flops = measure_attention(device)
    prof.dequant_bw = measure_dequant(device)
    prof.measured = tuple(sorted(set(prof.measured) | {"matmul_flops", "attn_flops", "dequant_bw"}))
    return prof
