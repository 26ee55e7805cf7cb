"""Benchmark of the NF4 hot path on one MI355X.

`value` is the throughput of one FLUX single-stream block's NF4 linears at 1024^2
(M = 4608 tokens: linear1 3072 -> 21504 and linear2 15360 -> 3072, weights N(0, 0.02)
NF4 blocksize 64, activations bf16 N(0, 1)), in TFLOP/s, inputs resident in HBM. A
step is linear1 + linear2 once; weights rotate over 8 distinct copies (512 MB of NF4,
above the 256 MB Infinity Cache).

The same JSON line carries:
  roofline      the fused GEMM kernel's FLOP/s from HIP-event durations of its launches
                against the 2.5 PFLOP/s dense bf16 MFMA peak;
  cpu_baseline  the reference's dequantize-then-torch path (the oracle's restatement of the torch
                NF4 decode + torch F.linear) on the host cores for the same two linears, the faster
                of fp32 and bf16; extra.cpu_baselines has every configuration (C1-C5) in both;
  extra         the other configurations: the 1536-token single linear, the 76 hoisted
                modulation GEMMs at M = 28 (HBM-bound, GB/s), the fused segments at M = 4608
                (GB/s), the library dequant + hipBLASLt path on the GPU for comparison, the fused
                attention against torch's SDPA at the FLUX shapes, and
                the full FLUX-dev-shaped step (batch 1 at 1024^2 and batch 4 at 512^2; s/step
                against the lower bound linear FLOP / peak + attention FLOP / peak + segment
                bytes / HBM peak).

Per-kernel figures are medians of HIP-event times over the timed steps (the roofline figure uses
the mean, as a kernel trace's average does). The default 30 warmup steps take the GPU past its
clock ramp under sustained load, and every configuration whose warm-up launches are short runs at least
80 ms of back-to-back launches before its timed ones.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-full-step] [--no-extra] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

METRIC = "NF4 linear TFLOP/s & HBM GB/s (% roofline); s/step FLUX 1024² on 1 GPU"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
D, MLP, M_1024 = 3072, 12288, 4608


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def nf4_weight(n, k, seed, dev):
    from selas_amd import codecs

    g = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    e = codecs.encode_nf4("w", w)
    del w
    return e


def bias(n, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(n, generator=g, device=dev) * 0.02).to(torch.bfloat16)


def act(m, k, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)


def lin(x, e, b=None):
    from selas_amd import codecs
    from selas_amd.linear import nf4_linear

    return nf4_linear(x, e.parts["packed"], e.parts["absmax"], 64, codecs.NF4_CODE, e.shape, b)


def sustain(fn, dev, min_s: float = 0.08) -> None:
    """Runs `fn` back to back for at least `min_s` of GPU time: under sustained load the GPU needs ~35 ms
    to settle its clock, and a short kernel's warm-up launches alone do not last that long."""
    t0 = time.perf_counter()
    while True:
        for _ in range(10):
            fn()
        torch.cuda.synchronize(dev)
        if time.perf_counter() - t0 >= min_s:
            return


class Timer:
    """HIP events on the current stream around individual launches."""

    def __init__(self):
        self.pairs: dict[str, list] = {}

    def start(self, name):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return name, e

    def stop(self, tok):
        name, e0 = tok
        e1 = torch.cuda.Event(enable_timing=True)
        e1.record()
        self.pairs.setdefault(name, []).append((e0, e1))

    def times_ms(self, name):
        return [a.elapsed_time(b) for a, b in self.pairs.get(name, [])]

    def mean_ms(self, name):
        ts = self.times_ms(name)
        return sum(ts) / max(1, len(ts))

    def median_ms(self, name):
        ts = sorted(self.times_ms(name))
        if not ts:
            return 0.0
        n = len(ts)
        return ts[n // 2] if n % 2 else 0.5 * (ts[n // 2 - 1] + ts[n // 2])


# --------------------------------------------------------------------------- config 2 (the value)


def bench_block_linears(dev, steps, warmup, copies=8):
    f1 = 2.0 * M_1024 * (3 * D + MLP) * D
    f2 = 2.0 * M_1024 * D * (D + MLP)
    w1 = [nf4_weight(3 * D + MLP, D, 100 + i, dev) for i in range(copies)]
    w2 = [nf4_weight(D, D + MLP, 200 + i, dev) for i in range(copies)]
    b1, b2 = bias(3 * D + MLP, 1, dev), bias(D, 2, dev)
    x1, x2 = act(M_1024, D, 2, dev), act(M_1024, D + MLP, 3, dev)
    for i in range(warmup):
        lin(x1, w1[i % copies], b1)
        lin(x2, w2[i % copies], b2)
    torch.cuda.synchronize(dev)
    tm = Timer()
    t0 = time.perf_counter()
    for i in range(steps):
        t = tm.start("linear1")
        lin(x1, w1[i % copies], b1)
        tm.stop(t)
        t = tm.start("linear2")
        lin(x2, w2[i % copies], b2)
        tm.stop(t)
    torch.cuda.synchronize(dev)
    wall = (time.perf_counter() - t0) / steps
    # The roofline figure uses the mean launch time (what a kernel trace's average reports); the
    # medians are listed beside it.
    k1, k2 = tm.mean_ms("linear1"), tm.mean_ms("linear2")
    nbytes = sum(e.nbytes for e in (w1[0], w2[0]))
    return {
        "flop_per_step": f1 + f2, "ms_per_step": wall * 1e3,
        "kernel_ms": {"linear1": k1, "linear2": k2},
        "kernel_ms_median": {"linear1": tm.median_ms("linear1"), "linear2": tm.median_ms("linear2")},
        "kernel_tflops": {"linear1": f1 / k1 / 1e9, "linear2": f2 / k2 / 1e9},
        "achieved_tflops": (f1 + f2) / (k1 + k2) / 1e9,
        "nf4_bytes_per_step": nbytes,
        "shapes": {"linear1": [M_1024, 3 * D + MLP, D], "linear2": [M_1024, D, D + MLP]},
    }


# --------------------------------------------------------------------------- extras


def bench_single_linear(dev, steps, warmup):
    m, n, k = 1536, 12288, 3072
    ws = [nf4_weight(n, k, 300 + i, dev) for i in range(8)]
    x = act(m, k, 1, dev)
    for i in range(warmup):
        lin(x, ws[i % 8])
    it = iter(range(1 << 30))
    sustain(lambda: lin(x, ws[next(it) % 8]), dev)  # ~130 us per launch: the warm-up count alone is a few ms
    tm = Timer()
    for i in range(steps):
        t = tm.start("l")
        lin(x, ws[i % 8])
        tm.stop(t)
    torch.cuda.synchronize(dev)
    ms = tm.median_ms("l")
    return {"shape": [m, n, k], "kernel_ms": ms, "tflops": 2.0 * m * n * k / ms / 1e9}


def bench_library_path(dev, steps, warmup):
    """The reference's GPU path for one block's linears: decode to bf16, then F.linear (hipBLASLt)."""
    from selas_amd import codecs

    w1, w2 = nf4_weight(3 * D + MLP, D, 100, dev), nf4_weight(D, D + MLP, 200, dev)
    x1, x2 = act(M_1024, D, 2, dev), act(M_1024, D + MLP, 3, dev)

    def run():
        a = codecs.decode("nf4", w1.parts, w1.meta, w1.shape, torch.bfloat16)
        torch.nn.functional.linear(x1, a)
        b = codecs.decode("nf4", w2.parts, w2.meta, w2.shape, torch.bfloat16)
        torch.nn.functional.linear(x2, b)

    for _ in range(warmup):
        run()
    sustain(run, dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize(dev)
    ms = (time.perf_counter() - t0) / steps * 1e3
    f = 2.0 * M_1024 * ((3 * D + MLP) * D + D * (D + MLP))
    # the GEMMs alone on pre-decoded weights
    a = codecs.decode("nf4", w1.parts, w1.meta, w1.shape, torch.bfloat16)
    b = codecs.decode("nf4", w2.parts, w2.meta, w2.shape, torch.bfloat16)
    tm = Timer()
    for _ in range(steps):
        t = tm.start("g")
        torch.nn.functional.linear(x1, a)
        torch.nn.functional.linear(x2, b)
        tm.stop(t)
    torch.cuda.synchronize(dev)
    g = tm.median_ms("g")
    return {"ms_per_step": ms, "tflops": f / ms / 1e9, "gemm_only_ms": g, "gemm_only_tflops": f / g / 1e9}


def bench_modulations(dev, steps, warmup):
    """76 hoisted adaLN linears at M = 28 (19 double blocks x img/txt 3072 -> 18432, 38 single 3072 -> 9216),
    76 distinct weights (1.8 GB of NF4, beyond the 256 MB Infinity Cache): one grouped launch, and one launch
    per linear."""
    from selas_amd import codecs
    from selas_amd.linear import GroupedPlan, nf4_linear_grouped

    s = 28
    ws = [nf4_weight(6 * D, D, 400 + i, dev) for i in range(38)] + [nf4_weight(3 * D, D, 500 + i, dev) for i in range(38)]
    bs = [bias(e.shape[0], 600 + i, dev) for i, e in enumerate(ws)]
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.nn.functional.silu(torch.randn(s, D, generator=g, device=dev)).to(torch.bfloat16)
    nbytes = sum(e.nbytes for e in ws) + sum(b.numel() * 2 for b in bs) + s * D * 2 + sum(s * e.shape[0] * 2 for e in ws)
    flops = sum(2.0 * s * e.shape[0] * D for e in ws)
    tuples = [(e.parts["packed"], e.parts["absmax"], 64, codecs.NF4_CODE, e.shape, b) for e, b in zip(ws, bs)]

    # One launch per linear straight through the C ABI (preallocated outputs), timed as one batch of
    # back-to-back launches: the Python wrapper's own time per call is about that of the kernel and would
    # leave the GPU idle between launches.
    from selas_amd import _lib

    lib, st, code = _lib.load(), _lib.stream(dev), _lib.code_array(codecs.NF4_CODE)
    ys = [torch.empty(s, e.shape[0], dtype=torch.bfloat16, device=dev) for e in ws]
    args = [(x.data_ptr(), s, D, D, e.parts["packed"].data_ptr(), e.parts["absmax"].data_ptr(), 64, code, e.shape[0],
             b.data_ptr(), y.data_ptr(), e.shape[0], _lib.BF16, None, 0, st) for e, b, y in zip(ws, bs, ys)]
    f = lib.selas_nf4_linear

    def run_each():
        for a in args:
            assert f(*a) == 0

    plan = GroupedPlan(tuples, s, dev)
    assert plan.supported
    for _ in range(max(2, warmup // 10)):
        run_each()
        nf4_linear_grouped(x, tuples)
        plan.run(x)
    torch.cuda.synchronize(dev)
    tm = Timer()
    reps = 5
    t = tm.start("gemv")
    for _ in range(reps):
        run_each()
    tm.stop(t)
    # the 38 double-block weights (18432 x 3072, 31.9 MB of NF4 each) alone, back to back
    t = tm.start("gemv_18432")
    for _ in range(reps):
        for a in args[:38]:
            f(*a)
    tm.stop(t)
    torch.cuda.synchronize(dev)
    assert torch.equal(ys[0], lin(x, ws[0], bs[0]))
    for _ in range(max(3, steps // 2)):
        t = tm.start("grouped_call")
        nf4_linear_grouped(x, tuples)
        tm.stop(t)
    sustain(lambda: plan.run(x), dev)
    for _ in range(max(5, steps)):
        t = tm.start("grouped_kernel")
        plan.run(x)
        tm.stop(t)
    torch.cuda.synchronize(dev)
    per = tm.mean_ms("gemv") / (reps * len(args))
    per18 = tm.mean_ms("gemv_18432") / (reps * 38)
    b18 = ws[0].nbytes + 6 * D * 2 + s * D * 2 + s * 6 * D * 2
    grp = tm.median_ms("grouped_kernel")
    call = tm.median_ms("grouped_call")
    assert all(torch.equal(a, b) for a, b in zip(plan.outs, ys))
    return {"launches": 76, "bytes": nbytes, "flops": flops, "grouped_kernel_ms": grp,
            "gbs_grouped": nbytes / grp / 1e6, "frac_hbm_grouped": nbytes / grp / 1e6 / PEAK_HBM_GBS,
            "grouped_call_ms": call, "per_linear_kernel_ms_mean": per, "gbs_per_linear": nbytes / (per * 76) / 1e6,
            "one_18432x3072": {"kernel_ms_mean": per18, "bytes": b18, "gbs": b18 / per18 / 1e6,
                               "frac_hbm": b18 / per18 / 1e6 / PEAK_HBM_GBS}}


def bench_int8_row(dev, steps, warmup, copies=8):
    """int8_row weights (selas convert --quant int8): the single block's linears at 1024^2 (tiled GEMM with
    the int8 operand), the same through decode + F.linear, and the 76 modulation linears at M = 28 (skinny
    kernel, one launch per linear; 3.2 GB of int8 weights)."""
    from selas_amd import codecs
    from selas_amd.linear import int8_row_linear

    def weight(n, k, seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        return codecs.encode_int8_row("w", torch.randn(n, k, generator=g, device=dev) * 0.02)

    def run(x, e, b=None):
        return int8_row_linear(x, e.parts["q"], e.parts["scale"], e.shape, b)

    f1 = 2.0 * M_1024 * (3 * D + MLP) * D
    f2 = 2.0 * M_1024 * D * (D + MLP)
    w1 = [weight(3 * D + MLP, D, 700 + i) for i in range(copies)]
    w2 = [weight(D, D + MLP, 800 + i) for i in range(copies)]
    b1, b2 = bias(3 * D + MLP, 1, dev), bias(D, 2, dev)
    x1, x2 = act(M_1024, D, 2, dev), act(M_1024, D + MLP, 3, dev)
    for i in range(warmup):
        run(x1, w1[i % copies], b1)
        run(x2, w2[i % copies], b2)
    it = iter(range(1 << 30))

    def pair():
        i = next(it)
        run(x1, w1[i % copies], b1)
        run(x2, w2[i % copies], b2)

    sustain(pair, dev)
    tm = Timer()
    for i in range(steps):
        t = tm.start("linear1")
        run(x1, w1[i % copies], b1)
        tm.stop(t)
        t = tm.start("linear2")
        run(x2, w2[i % copies], b2)
        tm.stop(t)
    torch.cuda.synchronize(dev)
    k1, k2 = tm.mean_ms("linear1"), tm.mean_ms("linear2")
    for i in range(max(3, steps // 5)):
        t = tm.start("library")
        torch.nn.functional.linear(x1, codecs.decode("int8_row", w1[i % copies].parts, {}, w1[0].shape,
                                                     torch.bfloat16), b1)
        torch.nn.functional.linear(x2, codecs.decode("int8_row", w2[i % copies].parts, {}, w2[0].shape,
                                                     torch.bfloat16), b2)
        tm.stop(t)
    torch.cuda.synchronize(dev)
    lib_ms = tm.median_ms("library")
    del w1, w2
    s = 28
    ws = [weight(6 * D, D, 900 + i) for i in range(38)] + [weight(3 * D, D, 1000 + i) for i in range(38)]
    bs = [bias(e.shape[0], 1100 + i, dev) for i, e in enumerate(ws)]
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.nn.functional.silu(torch.randn(s, D, generator=g, device=dev)).to(torch.bfloat16)
    nbytes = sum(e.nbytes for e in ws) + sum(b.numel() * 2 for b in bs) + s * D * 2 + sum(s * e.shape[0] * 2 for e in ws)
    # The 76 launches straight through the C ABI (preallocated outputs), timed as one batch: the
    # Python wrapper's own time per call is about that of the kernel and would leave the GPU idle.
    from selas_amd import _lib

    lib, st = _lib.load(), _lib.stream(dev)
    ys = [torch.empty(s, e.shape[0], dtype=torch.bfloat16, device=dev) for e in ws]
    args = [(x.data_ptr(), s, D, D, e.parts["q"].data_ptr(), e.parts["scale"].data_ptr(), e.shape[0], b.data_ptr(),
             y.data_ptr(), e.shape[0], _lib.BF16, None, 0, st) for e, b, y in zip(ws, bs, ys)]
    f = lib.selas_int8_row_linear
    for _ in range(max(2, warmup // 10)):
        for a in args:
            f(*a)
    torch.cuda.synchronize(dev)
    reps = 5
    t = tm.start("gemv")
    for _ in range(reps):
        for a in args:
            f(*a)
    tm.stop(t)
    torch.cuda.synchronize(dev)
    assert torch.equal(ys[0], run(x, ws[0], bs[0]))
    per = tm.mean_ms("gemv") / (reps * len(args))
    # All 76 in one launch of the streaming kernel.
    from selas_amd.linear import GroupedPlan

    plan = GroupedPlan([(e.parts["q"], e.parts["scale"], None, None, e.shape, b) for e, b in zip(ws, bs)], s, dev,
                       codec="int8_row")
    assert plan.supported
    for _ in range(max(2, warmup // 10)):
        plan.run(x)
    torch.cuda.synchronize(dev)
    for _ in range(max(5, steps)):
        t = tm.start("grouped")
        plan.run(x)
        tm.stop(t)
    torch.cuda.synchronize(dev)
    grp = tm.median_ms("grouped")
    assert all(torch.equal(a, b) for a, b in zip(plan.outs, ys))
    return {
        "block_linears": {"kernel_ms": {"linear1": k1, "linear2": k2},
                          "kernel_tflops": {"linear1": f1 / k1 / 1e9, "linear2": f2 / k2 / 1e9},
                          "achieved_tflops": (f1 + f2) / (k1 + k2) / 1e9,
                          "library_path_ms": lib_ms, "library_path_tflops": (f1 + f2) / lib_ms / 1e9},
        "modulations_m28": {"launches": 76, "bytes": nbytes, "grouped_kernel_ms": grp, "gbs_grouped": nbytes / grp / 1e6,
                            "frac_hbm_grouped": nbytes / grp / 1e6 / PEAK_HBM_GBS,
                            "per_linear_kernel_ms_mean": per, "per_linear_total_ms": per * 76,
                            "gbs_per_linear": nbytes / (per * 76) / 1e6},
    }


def bench_segments(dev, steps, warmup):
    from selas_amd.kernels import Kernels

    k = Kernels()
    g = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn(1, M_1024, D, generator=g, device=dev)
    mod = torch.randn(1, 3 * D, generator=g, device=dev) * 0.1
    sh, sc, gate = mod.float().unsqueeze(1).chunk(3, dim=-1)
    h = torch.randn(1, M_1024, 3 * D + MLP, generator=g, device=dev).to(torch.bfloat16)
    qkv = h[..., :3 * D]
    qs = 1 + 0.02 * torch.randn(128, generator=g, device=dev)
    ks = 1 + 0.02 * torch.randn(128, generator=g, device=dev)
    ang = torch.rand(M_1024, 64, generator=g, device=dev, dtype=torch.float64) * 50
    cos, sin = ang.cos().float(), ang.sin().float()
    y = torch.randn(1, M_1024, D, generator=g, device=dev).to(torch.bfloat16)
    attn = torch.randn(1, M_1024, D, generator=g, device=dev).to(torch.bfloat16)
    cases = {
        # name: (fn, algorithmic bytes per call)
        "mod_in": (lambda: k.mod_in(x, sh, sc, torch.bfloat16), M_1024 * D * (4 + 2) + 2 * D * 4),
        "qkv_single": (lambda: k.qkv_single(qkv, qs, ks, cos, sin, 24, torch.bfloat16),
                       M_1024 * 3 * D * 2 * 2 + 2 * M_1024 * 64 * 4),
        "gated_add": (lambda: k.gated_add(x, gate, y, False), M_1024 * D * (4 + 2 + 4) + D * 4),
        "attn_mlp": (lambda: k.attn_mlp(attn, h[..., 3 * D:]), M_1024 * (D + MLP) * 2 * 2),
    }
    # Each kernel runs for tens of microseconds, so a HIP-event pair around a single launch would add
    # its own few microseconds: the events bracket batches of back-to-back launches instead, and the
    # median batch time is divided by the batch size.
    batch = 20
    out = {}
    for name, (fn, nb) in cases.items():
        for _ in range(warmup):
            fn()
        sustain(fn, dev)
        tm = Timer()
        for _ in range(max(5, steps // 4)):
            t = tm.start(name)
            for _ in range(batch):
                fn()
            tm.stop(t)
        torch.cuda.synchronize(dev)
        ms = tm.median_ms(name) / batch
        out[name] = {"bytes": nb, "kernel_ms": ms, "gbs": nb / ms / 1e6, "frac_hbm": nb / ms / 1e6 / PEAK_HBM_GBS,
                     "timing": f"median of HIP-event batches of {batch} back-to-back launches"}
    return out


def segment_bytes(kind: str, cfg, l_img: int, l_txt: int, batch: int) -> float:
    """HBM bytes the fused segments of one block move per step (each tensor read or written once).

    Per token, D = hidden, F = mlp_hidden, Dh = head dim: mod_in reads x fp32 and writes bf16 (6D);
    attention prep reads q, k, v bf16 and writes them (12D) plus cos/sin (4 Dh); gated_add reads
    x fp32 and y bf16 and writes fp32 (10D); gated_add_mod also writes h bf16 (12D); gelu reads and
    writes F bf16 (4F); attn_mlp reads attn and mlp and writes the concat (4D + 4F)."""
    d, f, dh = cfg.hidden, cfg.mlp_hidden, cfg.hidden // cfg.heads
    tok = batch * (l_img + l_txt)
    if kind == "double":
        return tok * (6 * d + 12 * d + 4 * dh + 12 * d + 4 * f + 10 * d)
    if kind == "single":
        return tok * (6 * d + 12 * d + 4 * dh + 4 * d + 4 * f + 10 * d)
    return 0.0


def bench_attention(dev, steps, warmup):
    """The block attention at 1024^2 (B = 1, 24 heads x 128, L = 4608) and at 512^2 with batch 4 (L = 1536):
    the fused kernel (its launch alone, and the call with the value transpose) against the reference's
    SDPA + transpose/reshape (torch's flash backends)."""
    from selas_amd import _lib
    from selas_amd import flux as F
    from selas_amd.attention import attention, transpose_heads

    out = {}
    for name, b, l in (("b1_1024", 1, 4608), ("b4_512", 4, 1536)):
        g = torch.Generator(device=dev).manual_seed(6)
        q, k, v = (torch.randn(b, 24, l, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
        vt = transpose_heads(v)
        o = torch.empty(b, l, 24 * 128, dtype=torch.bfloat16, device=dev)

        def kernel():
            _lib.call("selas_attention", q.data_ptr(), k.data_ptr(), vt.data_ptr(), b, 24, l, 128, o.data_ptr(),
                      24 * 128, _lib.BF16, _lib.stream(dev))

        runs = {"kernel": kernel, "fused_call": lambda: attention(q, k, v), "sdpa": lambda: F.sdpa_attention(q, k, v)}
        flop = 4.0 * b * 24 * l * l * 128
        res = {"shape": [b, 24, l, 128], "flop": flop}
        for key, fn in runs.items():
            for _ in range(warmup):
                fn()
            sustain(fn, dev)
            tm = Timer()
            for _ in range(steps):
                t = tm.start(key)
                fn()
                tm.stop(t)
            torch.cuda.synchronize(dev)
            ms = tm.median_ms(key)
            res[key] = {"ms": ms, "tflops": flop / ms / 1e9}
        out[name] = res
    return out


def bench_full_step(dev, steps, warmup, batch=1, res=1024):
    """FLUX-dev-shaped step (19 double + 38 single blocks, all NF4 weights resident) at res^2 with
    `batch` images. Each image's 28-step modulations come from its own grouped skinny launch (outside
    the step time, as in the reference). Reports the median step time and the lower bound
    linear FLOP / peak + attention FLOP / peak + segment bytes / HBM peak."""
    from selas_amd import flux as F

    cfg = F.FluxConfig()
    t0 = time.perf_counter()
    model = F.RandomFlux(cfg, dev, torch.bfloat16, seed=0)
    torch.cuda.synchronize(dev)
    build_s = time.perf_counter() - t0
    g = torch.Generator(device=dev).manual_seed(5)
    n_steps = 28
    svs = [torch.nn.functional.silu(torch.randn(n_steps, 1, D, generator=g, device=dev)).to(torch.bfloat16)
           for _ in range(batch)]
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    per_image = [model.modulations(sv) for sv in svs]
    torch.cuda.synchronize(dev)
    prologue_s = (time.perf_counter() - t0) / batch
    mods = [torch.cat([m[j] for m in per_image], dim=1) for j in range(len(per_image[0]))]  # [S, B, kD]
    lt, grid = 512, res // 16
    txt = torch.randn(batch, lt, D, generator=g, device=dev)
    lat = torch.randn(batch, grid * grid, 64, generator=g, device=dev)
    fmod = (torch.randn(batch, 2 * D, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    ids = torch.cat((torch.zeros(lt, 3, device=dev), F.image_ids(grid, grid, dev)), dim=0)
    cos, sin = F.rope_tables(ids, cfg.axes_dim, cfg.theta)
    for s in range(warmup):
        model.step(lat, txt, [m[s] for m in mods], fmod, cos, sin)
    torch.cuda.synchronize(dev)
    tm = Timer()
    t0 = time.perf_counter()
    for s in range(steps):
        t = tm.start("step")
        v = model.step(lat, txt, [m[s % n_steps] for m in mods], fmod, cos, sin)
        tm.stop(t)
    torch.cuda.synchronize(dev)
    wall_s = (time.perf_counter() - t0) / steps
    step_s = tm.median_ms("step") / 1e3
    assert torch.isfinite(v).all()
    li = grid * grid
    blocks = (("double", 19), ("single", 38))
    lin_f = sum(F.unit_flops(kd, cfg, li, lt, batch)[0] * n for kd, n in blocks)
    att_f = sum(F.unit_flops(kd, cfg, li, lt, batch)[1] * n for kd, n in blocks)
    seg_b = sum(segment_bytes(kd, cfg, li, lt, batch) * n for kd, n in blocks) + batch * li * 6 * D
    bound_s = (lin_f + att_f) / (PEAK_BF16_TFLOPS * 1e12) + seg_b / (PEAK_HBM_GBS * 1e9)
    return {"batch": batch, "resolution": res, "tokens_per_image": li + lt, "steps": steps,
            "s_per_step": step_s, "s_per_step_wall": wall_s, "tflops": (lin_f + att_f) / step_s / 1e12,
            "linear_tflop": lin_f / 1e12, "attention_tflop": att_f / 1e12, "segment_gb": seg_b / 1e9,
            "lower_bound_s": bound_s, "frac_of_bound": bound_s / step_s,
            "prologue_s_per_image": prologue_s, "build_s": build_s, "nf4_resident_gb": model.nf4_bytes() / 1e9}


# --------------------------------------------------------------------------- CPU baseline


class CpuRefUnit:
    """The reference's CPU linear for one unit: every NF4 weight decoded on each call by the torch decode
    (selas/codecs.py:178-199, restated in the oracle) into the compute dtype, then F.linear in that dtype
    (selas/store.py:289-293). Parts are uniformly random codes and absmax: neither the decode's nor the
    GEMM's time depends on the values."""

    def __init__(self, shapes: dict, dt, seed: int):
        g = torch.Generator().manual_seed(seed)
        self.dt, self.w = dt, {}
        for name, (n, k) in shapes.items():
            packed = torch.randint(0, 256, (n * k // 2,), generator=g, dtype=torch.uint8)
            absmax = torch.rand(n * k // 64, generator=g) * 0.08 + 0.02
            bias = (torch.randn(n, generator=g) * 0.02).to(dt)
            self.w[name] = (packed, absmax, (n, k), bias)
        self.norms = {}

    def get(self, name, dtype=None):
        return self.norms.setdefault(name, torch.ones(128)).to(dtype or self.dt)

    def linear(self, x, prefix, dtype=None):
        from oracle import nf4 as onf4

        dt = dtype or self.dt
        packed, absmax, shape, bias = self.w[prefix]
        w = onf4.decode_torch(packed, absmax, 64, onf4.NF4_CODE, shape, dt)
        return torch.nn.functional.linear(x.to(dt), w, bias)


def _sdpa_cpu(q, k, v):
    """The reference's attention call (flux.py:135-138) on the CPU."""
    b, h, l, d = q.shape
    return torch.nn.functional.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(b, l, h * d)


def _timed(fn, reps: int = 1) -> float:
    fn()  # first call outside the timing (allocator, thread pool)
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps


def _rows_timed(run, total_rows: int, budget_s: float) -> tuple[float, int]:
    """Seconds for `run(rows)` at `total_rows`: timed in full when a 1/16 sample projects under
    `budget_s`, otherwise extrapolated linearly from the largest sample timed."""
    rows = max(1, total_rows // 16)
    t = _timed(lambda: run(rows))
    if t * total_rows / rows <= budget_s:
        return _timed(lambda: run(total_rows)), total_rows
    return t * total_rows / rows, rows


def cpu_baselines(budget_s: float = 6.0):
    """The reference's CPU path (dequantize-then-torch: the torch NF4 decode + F.linear, the eager segments)
    for every configuration, in fp32 and in bf16, on all host cores. C1-C3 are timed in full when that
    fits `budget_s` per run (otherwise on a row sample, extrapolated in rows); C4 on 4 of the 38 weights
    of each shape, extrapolated x38/4; C5 from one double and one single block at full shape plus img_in
    and the final layer, extrapolated x19 / x38."""
    from oracle import flux as OF
    from oracle import segments as S

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    out = {"cores": threads, "configs": {}}
    f32, bf16 = torch.float32, torch.bfloat16
    for dt in (f32, bf16):
        key = "fp32" if dt == f32 else "bf16"
        log(f"bench: cpu baseline {key}")
        res = {}
        # C1: 1536 x 12288 x 3072
        u = CpuRefUnit({"w": (4 * D, D)}, dt, 1)
        x = torch.randn(1536, D, generator=g).to(dt)
        t, rows = _rows_timed(lambda r: u.linear(x[:r], "w"), 1536, budget_s)
        res["c1_single_linear_1536"] = {"s": t, "tflops": 2.0 * 1536 * 4 * D * D / t / 1e12, "rows_timed": rows}
        # C2: linear1 + linear2 at M = 4608
        u = CpuRefUnit({"linear1": (3 * D + MLP, D), "linear2": (D, D + MLP)}, dt, 2)
        x1 = torch.randn(M_1024, D, generator=g).to(dt)
        x2 = torch.randn(M_1024, D + MLP, generator=g).to(dt)
        t1, r1 = _rows_timed(lambda r: u.linear(x1[:r], "linear1"), M_1024, budget_s)
        t2, r2 = _rows_timed(lambda r: u.linear(x2[:r], "linear2"), M_1024, budget_s)
        f2 = 2.0 * M_1024 * ((3 * D + MLP) * D + D * (D + MLP))
        res["c2_block_linears_1024"] = {"s": t1 + t2, "tflops": f2 / (t1 + t2) / 1e12, "rows_timed": [r1, r2]}
        # C3: the eager segments at M = 4608 (bytes as counted for the GPU kernels)
        xs = torch.randn(1, M_1024, D, generator=g)
        mod = torch.randn(1, 3 * D, generator=g) * 0.1
        sh, sc, gate = mod.unsqueeze(1).chunk(3, dim=-1)
        h = torch.randn(1, M_1024, 3 * D + MLP, generator=g).to(dt)
        qs, ks = 1 + 0.02 * torch.randn(128, generator=g), 1 + 0.02 * torch.randn(128, generator=g)
        ang = torch.rand(M_1024, 64, generator=g, dtype=torch.float64) * 50
        cos, sin = ang.cos().float(), ang.sin().float()
        y = torch.randn(1, M_1024, D, generator=g).to(dt)
        attn = torch.randn(1, M_1024, D, generator=g).to(dt)
        seg = {"mod_in": (lambda: S.mod_in(xs, sh, sc, dt), M_1024 * D * 6 + 2 * D * 4),
               "qkv_single": (lambda: S.qkv_single(h[..., :3 * D], qs, ks, cos, sin, 24, dt),
                              M_1024 * 3 * D * 2 * 2 + 2 * M_1024 * 64 * 4),
               "gated_add": (lambda: S.gated_add(xs, gate, y, False), M_1024 * D * 10 + D * 4),
               "attn_mlp": (lambda: S.attn_mlp(attn, h[..., 3 * D:]), M_1024 * (D + MLP) * 4)}
        res["c3_segments_4608"] = {}
        for name, (fn, nb) in seg.items():
            t = _timed(fn, 2)
            res["c3_segments_4608"][name] = {"s": t, "gbs": nb / t / 1e9}
        # C4: 76 modulation linears at M = 28 (4 weights of each shape timed)
        sv = torch.nn.functional.silu(torch.randn(28, D, generator=g)).to(dt)
        ud = CpuRefUnit({f"d{i}": (6 * D, D) for i in range(4)}, dt, 3)
        us = CpuRefUnit({f"s{i}": (3 * D, D) for i in range(4)}, dt, 4)
        td = _timed(lambda: [ud.linear(sv, f"d{i}") for i in range(4)])
        ts = _timed(lambda: [us.linear(sv, f"s{i}") for i in range(4)])
        t4 = (td + ts) * 38 / 4
        nb4 = 1876586496
        res["c4_modulations_m28"] = {"s": t4, "gbs": nb4 / t4 / 1e9, "sample": "4 + 4 of 38 + 38 weights"}
        # C5: one double + one single block at 1024^2 (B1), img_in and the final layer; x19 / x38
        cfg = OF.FluxConfig()
        dshapes = {}
        for st in ("img", "txt"):
            dshapes.update({f"{st}_attn.qkv": (3 * D, D), f"{st}_attn.proj": (D, D), f"{st}_mlp.0": (MLP, D),
                            f"{st}_mlp.2": (D, MLP)})
        du = CpuRefUnit(dshapes, dt, 5)
        su = CpuRefUnit({"linear1": (3 * D + MLP, D), "linear2": (D, D + MLP)}, dt, 6)
        gu = CpuRefUnit({"img_in": (D, 64), "final_layer.linear": (64, D)}, dt, 7)
        img = torch.randn(1, 4096, D, generator=g)
        txt = torch.randn(1, 512, D, generator=g)
        xs5 = torch.cat((txt, img), dim=1)
        ids = torch.cat((torch.zeros(512, 3), torch.stack(torch.meshgrid(torch.zeros(1), torch.arange(64.0),
                                                                          torch.arange(64.0), indexing="ij"),
                                                           -1).reshape(-1, 3)), dim=0)
        cos5, sin5 = S.rope_tables(ids, cfg.axes_dim, cfg.theta)
        dmod = (torch.randn(1, 12 * D, generator=g) * 0.1).to(dt)
        smod = (torch.randn(1, 3 * D, generator=g) * 0.1).to(dt)
        fmod = (torch.randn(1, 2 * D, generator=g) * 0.1).to(dt)
        lat = torch.randn(1, 4096, 64, generator=g)
        guard = dt == torch.float16
        k = S.OracleKernels
        tdb = _timed(lambda: OF.double_block(du, img, txt, dmod, cos5, sin5, cfg, dt, guard, k, _sdpa_cpu))
        tsb = _timed(lambda: OF.single_block(su, xs5, smod, cos5, sin5, cfg, dt, guard, k, _sdpa_cpu))
        tgl = _timed(lambda: (gu.linear(lat.to(dt), "img_in"), OF.final_layer(gu, img, fmod, dt, k)))
        t5 = 19 * tdb + 38 * tsb + tgl
        res["c5_full_step_1024_b1"] = {"s_per_step": t5, "double_block_s": tdb, "single_block_s": tsb,
                                       "globals_s": tgl, "tflops": 74.36e12 / t5 / 1e12,
                                       "sample": "one double + one single block at full shape, x19 / x38"}
        out["configs"][key] = res
    best = max(out["configs"].values(), key=lambda r: r["c2_block_linears_1024"]["tflops"])
    out["c2_best"] = {"value": best["c2_block_linears_1024"]["tflops"],
                      "dtype": "fp32" if best is out["configs"]["fp32"] else "bf16"}
    out["c5_best_s_per_step"] = min(r["c5_full_step_1024_b1"]["s_per_step"] for r in out["configs"].values())
    return out


# --------------------------------------------------------------------------- HBM traffic


TRAFFIC_FILE = ROOT / "profiles" / "nf4_gemm_block_linears_1024_traffic.md"


def committed_traffic():
    """HBM bytes per launch of the block-linear GEMM from the committed rocprofv3 --pmc summary (or None)."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def copy_calibration(dev, gib: float = 1.0, reps: int = 3):
    """A plain device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE counter readings."""
    n = int(gib * (1 << 30)) // 2
    a = torch.empty(n, dtype=torch.bfloat16, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize(dev)
    log(f"bench: copy calibration {reps} x {n * 2} bytes")
    del a, b


# --------------------------------------------------------------------------- main


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # Under sustained GEMM load the GPU takes ~60 launches (~35 ms) to reach its steady clock
    # (linear1: 985 TFLOP/s in the first 20 launches, 1,155 from the 60th on); 30 untimed steps
    # (60 launches) get past that ramp.
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-full-step", action="store_true",
                    help="skip the full FLUX-dev-shaped steps (batch 1 at 1024^2, batch 4 at 512^2)")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-calibration", action="store_true",
                    help="first run a 1 GiB device copy (reference for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: selas_amd has no multi-GPU path (asked for --gpus {a.gpus})",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda", 0)
    log(f"bench: {torch.cuda.get_device_name(dev)}")
    # The host-only CPU baselines run first, while the GPU is idle anyway; the GPU work follows, with the
    # headline measurement last, so that it runs on a GPU past its clock ramp under sustained load.
    cpu_all = None if a.no_cpu else cpu_baselines()
    if cpu_all is not None:
        for key, r in cpu_all["configs"].items():
            log(f"bench: cpu {key} on {cpu_all['cores']} cores: C1 {r['c1_single_linear_1536']['tflops']:.2f} "
                f"TFLOP/s, C2 {r['c2_block_linears_1024']['tflops']:.2f} TFLOP/s, C4 "
                f"{r['c4_modulations_m28']['gbs']:.1f} GB/s, C5 {r['c5_full_step_1024_b1']['s_per_step']:.1f} s/step")
    if a.traffic_calibration:
        copy_calibration(dev)
    extra = {}
    if not a.no_extra:
        extra["single_linear_1536"] = bench_single_linear(dev, a.steps, a.warmup)
        log(f"bench: single linear {extra['single_linear_1536']['tflops']:.1f} TFLOP/s")
        extra["modulations_m28"] = bench_modulations(dev, a.steps, a.warmup)
        mo = extra['modulations_m28']
        log(f"bench: modulations grouped {mo['gbs_grouped']:.0f} GB/s, per-linear {mo['gbs_per_linear']:.0f} GB/s")
        extra["segments_m4608"] = bench_segments(dev, a.steps, a.warmup)
        log(f"bench: segments {json.dumps({k: round(v['gbs']) for k, v in extra['segments_m4608'].items()})}")
        extra["library_path"] = bench_library_path(dev, a.steps, a.warmup)
        log(f"bench: library path {extra['library_path']['tflops']:.1f} TFLOP/s")
        extra["attention"] = bench_attention(dev, a.steps, a.warmup)
        extra["int8_row"] = bench_int8_row(dev, a.steps, a.warmup)
        i8 = extra["int8_row"]
        log(f"bench: int8_row block linears {i8['block_linears']['achieved_tflops']:.1f} TFLOP/s, "
            f"modulations grouped {i8['modulations_m28']['gbs_grouped']:.0f} GB/s, "
            f"per-linear {i8['modulations_m28']['gbs_per_linear']:.0f} GB/s")
        log("bench: attention " + ", ".join(f"{k}: fused {v['kernel']['tflops']:.0f} / SDPA {v['sdpa']['tflops']:.0f} TFLOP/s"
                                            for k, v in extra["attention"].items()))
    if not a.no_full_step:
        fs_steps = max(3, a.steps // 5)
        for key, batch, res_px in (("full_step_1024_b1", 1, 1024), ("full_step_512_b4", 4, 512)):
            extra[key] = bench_full_step(dev, fs_steps, 2, batch, res_px)
            r = extra[key]
            log(f"bench: full step B{batch} at {res_px}^2: {r['s_per_step']:.4f} s/step "
                f"(lower bound {r['lower_bound_s']:.4f} s, {100 * r['frac_of_bound']:.0f} %)")
        if cpu_all is not None:
            fs = extra["full_step_1024_b1"]
            fs["cpu_s_per_step"] = cpu_all["c5_best_s_per_step"]
            fs["speedup_vs_cpu"] = cpu_all["c5_best_s_per_step"] / fs["s_per_step"]
            log(f"bench: full step B1 at 1024^2: {fs['s_per_step']:.4f} s/step on the GPU, "
                f"{fs['cpu_s_per_step']:.1f} s/step on {cpu_all['cores']} CPU cores")
    res = bench_block_linears(dev, a.steps, a.warmup)
    log(f"bench: block linears {res['kernel_tflops']}")
    extra["block_linears"] = res
    cpu = None
    if cpu_all is not None:
        extra["cpu_baselines"] = cpu_all
        cpu = {"value": cpu_all["c2_best"]["value"], "unit": "TFLOP/s", "cores": cpu_all["cores"], "kind": "port",
               "sample": f"the reference's dequantize-then-F.linear path on the host (the oracle's restatement of "
                         f"the torch NF4 decode, torch F.linear) for linear1 + linear2 at M = 4608, "
                         f"{cpu_all['c2_best']['dtype']} (the faster of fp32 and bf16), all rows; every config "
                         f"in extra.cpu_baselines"}
    achieved = res["achieved_tflops"]
    line = {
        "metric": METRIC,
        "value": res["flop_per_step"] / (res["ms_per_step"] / 1e3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "FLUX single-stream block NF4 linears at 1024^2: M=4608, linear1 3072->21504 + "
                               "linear2 15360->3072, NF4 blocksize 64, bf16 activations", "tokens": M_1024,
                   "hidden": D, "mlp_hidden": MLP, "blocksize": 64, "weight_copies": 8},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": committed_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
