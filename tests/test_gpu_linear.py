"""Quantized linear on the GPU (fused-dequant MFMA GEMM for M > 32, skinny dequant-GEMM for
M <= 32) against the oracle: x @ decode(W).T + b with fp32 accumulation in fp64 on the CPU.

Tolerance (stated by the path's contract): max |y - ref| <= 1e-2 * max |ref| and relative
L2 error <= 4e-3. The fused GEMM's weight operand is additionally checked bit-exact with
one-hot inputs (x = e_k gives y[:, n] = W_bf16[n, k] exactly).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4 as onf4
from selas_amd import _lib, codecs
from selas_amd.linear import UnitView, nf4_linear

from .conftest import seeded

pytestmark = pytest.mark.gpu

MAX_REL, L2_REL = 1e-2, 4e-3


def make_weight(n, k, seed, dev, bs=64, scale=0.02):
    w = torch.randn(n, k, generator=seeded(seed)) * scale
    p, a = onf4.encode(w.numpy(), bs)
    ref = torch.from_numpy(onf4.bf16_to_f32(onf4.decode(p, a, bs, out=onf4.BF16))).view(n, k)
    return torch.from_numpy(p).to(dev), torch.from_numpy(a).to(dev), ref


def oracle_linear(x, w_ref, bias=None):
    y = x.double().cpu() @ w_ref.double().t()
    if bias is not None:
        y = y + bias.double().cpu()
    return y


def check_close(y, ref):
    y = y.double().cpu()
    err = (y - ref).abs().max().item()
    assert err <= MAX_REL * ref.abs().max().item(), f"max abs err {err} vs max {ref.abs().max().item()}"
    rel = ((y - ref).norm() / ref.norm()).item()
    assert rel <= L2_REL, f"relative L2 {rel}"


@pytest.mark.parametrize("m,n,k", [(1, 64, 64), (7, 100, 128), (28, 9216, 3072), (32, 192, 3072), (3, 4160, 640)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_skinny_path(dev, m, n, k, with_bias):
    p, a, w_ref = make_weight(n, k, m + n, dev)
    x = (torch.randn(m, k, generator=seeded(1)).to(torch.bfloat16)).to(dev)
    b = (torch.randn(n, generator=seeded(2)) * 0.02).to(torch.bfloat16).to(dev) if with_bias else None
    y = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b)
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    check_close(y, oracle_linear(x, w_ref, b))


@pytest.mark.parametrize("m,n,k", [(33, 64, 64), (100, 96, 128), (256, 256, 3072), (257, 300, 192),
                                   (513, 3072, 640), (1536, 512, 3072)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_tiled_path(dev, m, n, k, with_bias):
    p, a, w_ref = make_weight(n, k, m + n + k, dev)
    x = torch.randn(m, k, generator=seeded(3)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(4)) * 0.02).to(torch.bfloat16).to(dev) if with_bias else None
    y = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b)
    check_close(y, oracle_linear(x, w_ref, b))


def test_tiled_operand_is_the_reference_decode_bit_for_bit(dev):
    n, k, m = 320, 640, 96
    p, a, w_ref = make_weight(n, k, 7, dev)
    ks = torch.randint(0, k, (m,), generator=seeded(8))
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    x[torch.arange(m), ks] = 1.0
    y = nf4_linear(x.to(dev), p, a, 64, codecs.NF4_CODE, (n, k)).float().cpu()
    assert torch.equal(y, w_ref[:, ks].t())


@pytest.mark.parametrize("n,k", [(192, 256), (96, 3072), (64, 1024)])
def test_skinny_operand_within_one_rounding(dev, n, k):
    m = 16
    p, a, w_ref = make_weight(n, k, 9, dev)
    ks = torch.randint(0, k, (m,), generator=seeded(10))
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    x[torch.arange(m), ks] = 1.0
    y = nf4_linear(x.to(dev), p, a, 64, codecs.NF4_CODE, (n, k)).float().cpu()
    ref = w_ref[:, ks].t()
    assert ((y - ref).abs() <= 2.0 ** -7 * ref.abs()).all()


def test_skinny_rows_of_any_magnitude(dev):
    # The streaming skinny kernel rescales each row of x by a power of two before
    # its fp16 products: rows far from 1, an all-zero row and a row with one huge
    # entry must each match the oracle relative to that row alone.
    n, k = 256, 3072
    p, a, w_ref = make_weight(n, k, 31, dev)
    b = (torch.randn(n, generator=seeded(33)) * 0.02).to(torch.bfloat16)
    x = torch.randn(6, k, generator=seeded(32))
    x[0] *= 2.0 ** -60
    x[1] *= 2.0 ** 60
    x[2] = 0.0
    x[3, 17] = 3.0e38
    x[4] = x[4].abs() + 1.0  # all positive: coherent sums
    x = x.to(torch.bfloat16)
    y = nf4_linear(x.to(dev), p, a, 64, codecs.NF4_CODE, (n, k), b.to(dev))
    ref = oracle_linear(x, w_ref, b)
    for r in range(6):
        check_close(y[r:r + 1], ref[r:r + 1])


def test_strided_and_batched_inputs(dev):
    n, k = 256, 192
    p, a, w_ref = make_weight(n, k, 11, dev)
    base = torch.randn(2, 70, k + 64, generator=seeded(12)).to(torch.bfloat16).to(dev)
    x = base[:, 3:, 32:32 + k]  # [2, 67, k] with row stride k+64, batch stride 70*(k+64)
    y = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k))
    assert y.shape == (2, 67, n)
    check_close(y.reshape(-1, n), oracle_linear(x.reshape(-1, k), w_ref))


def test_unsupported_shapes_fall_back_to_decode_and_library_gemm(dev):
    n, k = 96, 96  # K % 64 != 0 with blocksize 32
    p, a, w_ref = make_weight(n, k, 13, dev, bs=32)
    x = torch.randn(40, k, generator=seeded(14)).to(torch.bfloat16).to(dev)
    y = nf4_linear(x, p, a, 32, codecs.NF4_CODE, (n, k))
    check_close(y, oracle_linear(x, w_ref))


def test_deterministic_across_calls(dev):
    n, k = 3072, 3072
    p, a, _ = make_weight(n, k, 15, dev)
    for m in (28, 300):
        x = torch.randn(m, k, generator=seeded(16)).to(torch.bfloat16).to(dev)
        y1 = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k))
        y2 = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k))
        assert torch.equal(y1, y2)


def test_unit_view_linear(dev):
    n, k = 128, 256
    w = torch.randn(n, k, generator=seeded(17)) * 0.02
    e = codecs.encode_nf4("lin.weight", w.to(dev))
    b = codecs.encode_raw("lin.bias", (torch.randn(n, generator=seeded(18)) * 0.02).to(dev), torch.bfloat16)
    view = UnitView({"lin.weight": e, "lin.bias": b}, torch.bfloat16)
    x = torch.randn(1, 80, k, generator=seeded(19)).to(torch.bfloat16).to(dev)
    y = view.linear(x, "lin")
    w_ref = view.get("lin.weight").float().cpu()
    check_close(y.reshape(-1, n), oracle_linear(x.reshape(-1, k), w_ref, b.parts["data"]))
    assert view.get("lin.bias").data_ptr() == b.parts["data"].data_ptr()


def test_full_size_single_linear(dev):
    # config 1: W 12288x3072 ~ N(0, 0.02) seed 0, X 1536x3072 bf16 ~ N(0, 1) seed 1; rows sampled for the oracle
    n, k, m = 12288, 3072, 1536
    w = torch.randn(n, k, generator=seeded(0)) * 0.02
    e = codecs.encode_nf4("w", w.to(dev))
    x = torch.randn(m, k, generator=seeded(1)).to(torch.bfloat16).to(dev)
    y = nf4_linear(x, e.parts["packed"], e.parts["absmax"], 64, codecs.NF4_CODE, (n, k))
    dec = onf4.decode(e.parts["packed"].cpu().numpy(), e.parts["absmax"].cpu().numpy(), 64, out=onf4.BF16)
    w_ref = torch.from_numpy(onf4.bf16_to_f32(dec)).view(n, k)
    rows = torch.randint(0, m, (64,), generator=seeded(2))
    check_close(y[rows], oracle_linear(x[rows], w_ref))
    assert torch.isfinite(y).all()


@pytest.mark.parametrize("k", [1024, 2048, 3072])
def test_streaming_skinny_every_m_with_strided_x(dev, k):
    # The streaming kernel copies each wave's slice of x through LDS, 32 rows x 128 bytes per round, rows past M
    # repeating row M-1. Every M from 1 to 32, with x a column slice of a wider buffer (row stride k + 192).
    n = 160
    p, a, w_ref = make_weight(n, k, 7 + k, dev)
    wide = torch.randn(32, k + 192, generator=seeded(k)).to(torch.bfloat16).to(dev)
    for m in range(1, 33):
        x = wide[:m, 64:64 + k]
        assert x.stride() == (k + 192, 1)
        y = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), None)
        check_close(y, oracle_linear(x, w_ref))
        assert torch.equal(y, nf4_linear(x.contiguous(), p, a, 64, codecs.NF4_CODE, (n, k), None))


def test_grouped_skinny_equals_one_by_one(dev):
    from selas_amd.linear import nf4_linear_grouped

    shapes = [(3072 * 6, 3072), (192, 3072), (64, 3072), (100, 3072), (3072 * 3, 3072)]
    ws = []
    for i, (n, k) in enumerate(shapes):
        p, a, w_ref = make_weight(n, k, 40 + i, dev)
        b = (torch.randn(n, generator=seeded(50 + i)) * 0.02).to(torch.bfloat16).to(dev) if i % 2 == 0 else None
        ws.append(((p, a, 64, codecs.NF4_CODE, (n, k), b), w_ref))
    for m in (1, 28, 32):
        x = torch.nn.functional.silu(torch.randn(m, 1, 3072, generator=seeded(m))).to(torch.bfloat16).to(dev)
        ys = nf4_linear_grouped(x, [w for w, _ in ws])
        for (w, w_ref), y in zip(ws, ys):
            alone = nf4_linear(x, *w)
            assert y.shape == alone.shape == (m, 1, w[4][0])
            assert torch.equal(y, alone)  # same bits as the per-linear call
            check_close(y.reshape(m, -1), oracle_linear(x.reshape(m, -1), w_ref, w[5]))


def test_batched_equals_one_by_one(dev):
    from selas_amd.linear import nf4_linear_batched

    shapes = [(300, 256, 3072), (64, 192, 640), (512, 320, 1024), (100, 64, 64), (1000, 96, 128)]
    probs, refs = [], []
    for i, (m, n, k) in enumerate(shapes):
        p, a, w_ref = make_weight(n, k, 70 + i, dev)
        x = torch.randn(m, k, generator=seeded(80 + i)).to(torch.bfloat16).to(dev)
        b = (torch.randn(n, generator=seeded(90 + i)) * 0.02).to(torch.bfloat16).to(dev) if i % 2 else None
        probs.append((x, p, a, 64, codecs.NF4_CODE, (n, k), b))
        refs.append(w_ref)
    ys = nf4_linear_batched(probs)  # five problems: a launch of four, then one
    for prob, w_ref, y in zip(probs, refs, ys):
        assert torch.equal(y, nf4_linear(*prob))  # same bits as the call alone
        check_close(y, oracle_linear(prob[0], w_ref, prob[6]))
    # a skinny problem in the batch: everything runs one by one, same results
    xs = torch.randn(8, 3072, generator=seeded(99)).to(torch.bfloat16).to(dev)
    mixed = [probs[0], (xs,) + probs[0][1:]]
    y0, y1 = nf4_linear_batched(mixed)
    assert torch.equal(y0, nf4_linear(*probs[0])) and torch.equal(y1, nf4_linear(*mixed[1]))



@pytest.mark.parametrize("m,n,k,gc", [(300, 1280, 640, 512), (100, 256, 128, 256), (513, 2304, 3072, 1792),
                                      (40, 768, 64, 512), (20, 512, 256, 256), (64, 300, 128, 45)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gelu_epilogue_equals_linear_then_gelu(dev, m, n, k, gc, with_bias):
    # The last gc output columns GELU'd in the GEMM epilogue, written into a strided destination, against
    # nf4_linear followed by the GELU segment kernel: the same bits. (20 rows: skinny path; 300 - 45 plain columns,
    # not a multiple of 256: both take the composed fallback.)
    from selas_amd.kernels import Kernels
    from selas_amd.linear import nf4_linear_gelu

    p, a, w_ref = make_weight(n, k, m + n + gc, dev)
    x = torch.randn(m, k, generator=seeded(41)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(42)) * 0.02).to(torch.bfloat16).to(dev) if with_bias else None
    wide = torch.zeros(m, gc + 64, dtype=torch.bfloat16, device=dev)
    ((y, g),) = nf4_linear_gelu([(x, p, a, 64, codecs.NF4_CODE, (n, k), b, gc, wide[:, 32:32 + gc])])
    full = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b)
    assert torch.equal(g, Kernels().gelu(full[:, n - gc:]))
    assert (y is None) == (gc == n) and (y is None or torch.equal(y, full[:, :n - gc]))
    assert torch.count_nonzero(wide[:, :32]) == 0 and torch.count_nonzero(wide[:, 32 + gc:]) == 0
    check_close(full, oracle_linear(x, w_ref, b))


def test_split_tail_with_gelu_columns(dev):
    # M = 16640, N = 1024, K = 2048: 65 x 4 = 260 tiles of 256 x 256, one round plus 4 (the last row slab,
    # rows 16384-16639). On 256 CUs those 4 run as 8 K ranges each, and a second kernel adds the ranges and
    # finishes them: bias, rounding and, for the last 512 columns, GELU. The GELU columns must equal the
    # plain output of the same launch through the GELU segment bit for bit, the whole tiles must equal a
    # launch of their rows alone, and everything must match the oracle.
    from selas_amd.kernels import Kernels
    from selas_amd.linear import nf4_linear_gelu

    m, n, k, gc = 16640, 1024, 2048, 512
    p, a, w_ref = make_weight(n, k, 81, dev)
    x = torch.randn(m, k, generator=seeded(82)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(83)) * 0.02).to(torch.bfloat16).to(dev)
    ((y, g),) = nf4_linear_gelu([(x, p, a, 64, codecs.NF4_CODE, (n, k), b, gc, None)])
    full = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b)
    assert torch.equal(y, full[:, :n - gc]) and torch.equal(g, Kernels().gelu(full[:, n - gc:]))
    assert torch.equal(nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b), full)
    assert torch.equal(full[:16384], nf4_linear(x[:16384], p, a, 64, codecs.NF4_CODE, (n, k), b))
    tail = full[16384:].double()
    alone = nf4_linear(x[16384:], p, a, 64, codecs.NF4_CODE, (n, k), b).double()
    assert ((tail - alone).norm() / alone.norm()).item() < 1e-4
    rows = torch.cat([torch.randint(0, 16384, (96,), generator=seeded(84)), torch.arange(16384, m, 4)])
    check_close(full[rows], oracle_linear(x[rows], w_ref, b))


@pytest.mark.parametrize("m,n,k", [(16384, 1024, 2048), (16640, 1024, 2048), (1536, 12288, 128)])
def test_bits_do_not_depend_on_concurrent_kernels(dev, m, n, k):
    # The tiled GEMM run on two streams at once, and beside an unrelated kernel on another stream, gives
    # the bits of the same launches alone. K = 2048 is 32 K blocks, two past the unrolled loop of three: a
    # wait there counted loads that the compiler had deleted, and the last block's x tile could still be
    # in flight when it was read, which showed only when another kernel slowed the loads down (16384
    # rows: 256 tiles in one round). 16640 rows also split the last round's 4 tiles over K, whose partial
    # tiles live in a workspace each call allocates. 1536 x 12288 x 128 runs 192-row tiles with two blocks after
    # the (empty) loop.
    p, a, _ = make_weight(n, k, 91, dev)
    xs = [torch.randn(m, k, generator=seeded(92 + i)).to(torch.bfloat16).to(dev) for i in range(2)]
    ref = [nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), None) for x in xs]
    big = torch.randn(64 << 20, device=dev)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    outs = [[], []]
    for _ in range(4):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                outs[i].append(nf4_linear(xs[i], p, a, 64, codecs.NF4_CODE, (n, k), None))
    for _ in range(4):
        with torch.cuda.stream(streams[0]):
            outs[0].append(nf4_linear(xs[0], p, a, 64, codecs.NF4_CODE, (n, k), None))
        with torch.cuda.stream(streams[1]):
            big.mul_(1.0)
    torch.cuda.synchronize()
    for i in range(2):
        for y in outs[i]:
            assert torch.equal(y, ref[i])


def test_split_launches_on_many_streams(dev):
    # The split plan and its workspace come from the shapes alone (the caller allocates the workspace per
    # call), so every stream gives the same bits: 12 streams at once, with the default stream's result
    # (M = 16640, N = 1024, K = 2048: the last row slab's 4 tiles run as 8 K ranges each on 256 CUs).
    m, n, k = 16640, 1024, 2048
    assert _lib.workspace_bytes(_lib.CODEC_NF4, ((m, k, n),), dev) == 4 * 8 * 256 * 1024
    p, a, w_ref = make_weight(n, k, 101, dev)
    x = torch.randn(m, k, generator=seeded(102)).to(torch.bfloat16).to(dev)
    ref = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), None)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(dev) for _ in range(12)]
    outs = []
    for st in streams:
        with torch.cuda.stream(st):
            outs.append(nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), None))
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(y, ref)
    # the split tiles sum K in another order than a launch of their rows alone (one round, unsplit)
    alone = nf4_linear(x[16384:], p, a, 64, codecs.NF4_CODE, (n, k), None)
    d = (ref[16384:].double() - alone.double()).norm() / alone.double().norm()
    assert d.item() < 1e-4
    rows = torch.arange(16384, m, 8)
    check_close(outs[-1][rows], oracle_linear(x[rows], w_ref, None))


def test_split_launch_in_a_captured_graph(dev):
    # A split shape captured in a HIP graph (its workspace comes from the graph's memory pool) and replayed
    # several times, with eager work between the replays: every replay gives the eager launch's bits.
    m, n, k = 16640, 1024, 2048
    p, a, _ = make_weight(n, k, 103, dev)
    x = torch.randn(m, k, generator=seeded(104)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(105)) * 0.02).to(torch.bfloat16).to(dev)
    eager = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm the wrapper's caches outside capture
        nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b)
    for i in range(4):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(y, eager), i
        other = nf4_linear(x[:4096], p, a, 64, codecs.NF4_CODE, (n, k), b)  # eager work between replays
        torch.cuda.synchronize(dev)
        assert torch.equal(other, eager[:4096])


def test_tile_height_does_not_change_the_bits(dev):
    # M = 2048, N = 8192 runs 256-row tiles (256 tiles, one round); its first 300 rows alone run
    # 192-row tiles (one round either way, fewer rows per tile). Every output sums K in the same
    # order, so the bits agree; both are checked against the oracle.
    n, k = 8192, 256
    p, a, w_ref = make_weight(n, k, 61, dev)
    x = torch.randn(2048, k, generator=seeded(62)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(63)) * 0.02).to(torch.bfloat16).to(dev)
    big = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b)
    small = nf4_linear(x[:300], p, a, 64, codecs.NF4_CODE, (n, k), b)
    assert torch.equal(big[:300], small)
    rows = torch.randint(0, 2048, (128,), generator=seeded(64))
    check_close(big[rows], oracle_linear(x[rows], w_ref, b))
    check_close(small, oracle_linear(x[:300], w_ref, b))


@pytest.mark.parametrize("n", [1024, 1000])
def test_bias_alignment_does_not_change_the_bits(dev, n):
    # The tiled kernel brings a 16-byte aligned bias into LDS by DMA and reads any other bias
    # with 2-byte loads; a bias view at a 2-byte offset must give the same bits as an aligned
    # copy. N = 1000 leaves the last column tile partial (per-element bias there).
    k = 256
    p, a, w_ref = make_weight(n, k, 71, dev)
    x = torch.randn(600, k, generator=seeded(72)).to(torch.bfloat16).to(dev)
    buf = (torch.randn(n + 8, generator=seeded(73)) * 0.02).to(torch.bfloat16).to(dev)
    b_odd = buf[1:n + 1]
    assert b_odd.data_ptr() % 16 != 0
    b_al = b_odd.clone()
    assert b_al.data_ptr() % 16 == 0
    y_odd = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b_odd)
    y_al = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b_al)
    assert torch.equal(y_odd, y_al)
    check_close(y_al, oracle_linear(x, w_ref, b_al))
    # no bias: the kernel reads an empty range (zeros)
    y_none = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), None)
    check_close(y_none, oracle_linear(x, w_ref, None))


def test_224_row_tiles_give_the_same_bits(dev):
    # On a 256-CU GPU, M = 448, N = 44032 (172 column tiles) runs 224-row tiles: 344 tiles in two
    # rounds, where 192-row tiles would need three; its 2048-row superset runs 256-row tiles. The
    # shared rows must agree bit for bit whichever heights the launches pick.
    n, k = 44032, 64
    p, a, w_ref = make_weight(n, k, 65, dev)
    x = torch.randn(2048, k, generator=seeded(66)).to(torch.bfloat16).to(dev)
    big = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k))
    small = nf4_linear(x[:448], p, a, 64, codecs.NF4_CODE, (n, k))
    assert torch.equal(big[:448], small)
    rows = torch.randint(0, 448, (64,), generator=seeded(67))
    check_close(small[rows], oracle_linear(x[rows], w_ref, None))


_RNG_SHAPES = [(int(m), int(n), int(k)) for m, n, k in zip(
    torch.randint(33, 700, (10,), generator=seeded(2024)).tolist(),
    (torch.randint(1, 21, (10,), generator=seeded(2025)) * 64).tolist(),
    (torch.randint(1, 17, (10,), generator=seeded(2026)) * 64).tolist())]


@pytest.mark.parametrize("m,n,k", _RNG_SHAPES)
def test_seeded_random_shapes(dev, m, n, k):
    # Shapes drawn once from a seeded generator (M 33-699, N and K multiples of 64): both tile
    # heights, partial row and column tiles, bias on odd draws.
    p, a, w_ref = make_weight(n, k, m * 7 + n, dev)
    x = torch.randn(m, k, generator=seeded(m + k)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(n)) * 0.02).to(torch.bfloat16).to(dev) if m % 2 else None
    check_close(nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), b), oracle_linear(x, w_ref, b))


def test_seeded_random_shapes_beside_another_kernel(dev):
    # The seeded shapes (K from 1 to 16 blocks: every remainder of the three-block loop) again, each run
    # four times while an elementwise kernel streams 256 MB on a second stream: the same bits as alone.
    big = torch.randn(64 << 20, device=dev)
    other = torch.cuda.Stream(dev)
    for m, n, k in _RNG_SHAPES:
        p, a, _ = make_weight(n, k, m * 7 + n, dev)
        x = torch.randn(m * 8, k, generator=seeded(m + k)).to(torch.bfloat16).to(dev)
        ref = nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), None)
        torch.cuda.synchronize()
        outs = []
        for _ in range(4):
            with torch.cuda.stream(other):
                big.mul_(1.0)
            outs.append(nf4_linear(x, p, a, 64, codecs.NF4_CODE, (n, k), None))
        torch.cuda.synchronize()
        assert all(torch.equal(y, ref) for y in outs), (m * 8, n, k)
