"""int8_row codec and linear on the GPU against the oracle (oracle/int8_row.py).

Decode and encode are bit-exact. The linears are checked against x @ decode(W).T + b
in fp64 on the CPU with the path's tolerance: max |y - ref| <= 1e-2 * max |ref| and
relative L2 <= 4e-3. The tiled GEMM's operand is additionally bit-exact (one-hot
inputs read it back); the skinny kernel multiplies by q exactly and scales the row
sums, so its one-hot readback is within one bf16 rounding of the decoded weight.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import int8_row as oi8
from oracle import nf4 as onf4
from selas_amd import _lib, codecs
from selas_amd.linear import UnitView, int8_row_linear, int8_row_linear_batched, int8_row_linear_gelu

from .conftest import seeded

pytestmark = pytest.mark.gpu

MAX_REL, L2_REL = 1e-2, 4e-3
OUT = {torch.bfloat16: oi8.BF16, torch.float16: oi8.F16, torch.float32: oi8.F32}


def check_close(y, ref):
    y = y.double().cpu()
    err = (y - ref).abs().max().item()
    assert err <= MAX_REL * ref.abs().max().item(), f"max abs err {err} vs max {ref.abs().max().item()}"
    rel = ((y - ref).norm() / ref.norm()).item()
    assert rel <= L2_REL, f"relative L2 {rel}"


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def make_weight(n, k, seed, dev, scale=0.02):
    w = torch.randn(n, k, generator=seeded(seed)) * scale
    q, s = oi8.encode(w.numpy())
    ref = torch.from_numpy(onf4.bf16_to_f32(oi8.decode(q, s, oi8.BF16))).view(n, k)
    return torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), ref


def oracle_linear(x, w_ref, bias=None):
    y = x.double().cpu() @ w_ref.double().t()
    return y if bias is None else y + bias.double().cpu()


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(64, 256), (33, 100), (5, 3, 48), (1, 16)])
def test_decode_bit_exact(dev, dt, shape):
    g = seeded(sum(shape))
    q = torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)  # -128 as imported data may hold it
    s = torch.rand(shape[0], generator=g) * 0.1 + 1e-5
    s[0] = 1.0 + 3 * 2.0 ** -10  # rounds to 1 in bf16
    out = codecs.decode("int8_row", {"q": q.to(dev), "scale": s.to(dev)}, {}, shape, dt)
    assert out.shape == shape and out.dtype == dt
    assert np.array_equal(bits(out), oi8.decode(q.numpy(), s.numpy(), OUT[dt]))


@pytest.mark.parametrize("shape", [(64, 256), (37, 100), (4, 3, 40), (3, 5000)])
def test_encode_bit_exact(dev, shape):
    w = torch.randn(*shape, generator=seeded(shape[0])) * torch.rand(shape[0], *([1] * (len(shape) - 1)),
                                                                      generator=seeded(1)) * 3
    w[1] *= 50  # an outlier row
    w[2] = 0.0  # a zero row: scale 1
    if shape[-1] >= 8:  # exact ties: a row of k + 1/2 with scale 1
        w[0].view(-1)[:8] = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -127.0])
        w[0].view(-1)[8:] = 0.25
    e = codecs.encode_int8_row("w", w.to(dev))
    q_ref, s_ref = oi8.encode(w.numpy())
    assert e.codec == "int8_row" and e.shape == shape and e.parts["q"].shape == shape
    assert np.array_equal(e.parts["q"].cpu().numpy(), q_ref)
    assert np.array_equal(e.parts["scale"].cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_encode_cpu_tensor_returns_cpu_parts_and_rejects_vectors(dev):
    w = torch.randn(16, 64, generator=seeded(3))
    e = codecs.encode_int8_row("w", w)
    assert e.parts["q"].device.type == "cpu" and e.parts["scale"].device.type == "cpu"
    with pytest.raises(ValueError):
        codecs.encode_int8_row("v", torch.ones(8))


@pytest.mark.parametrize("m,n,k", [(1, 64, 64), (7, 100, 128), (28, 18432, 3072), (32, 192, 3072), (3, 4160, 640)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_skinny_path(dev, m, n, k, with_bias):
    q, s, w_ref = make_weight(n, k, m + n, dev)
    x = torch.nn.functional.silu(torch.randn(m, k, generator=seeded(1))).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(2)) * 0.02).to(torch.bfloat16).to(dev) if with_bias else None
    y = int8_row_linear(x, q, s, (n, k), b)
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    check_close(y, oracle_linear(x, w_ref, b))


@pytest.mark.parametrize("m,n,k", [(33, 64, 64), (100, 96, 128), (257, 300, 192), (513, 3072, 640),
                                   (1536, 512, 3072)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_tiled_path(dev, m, n, k, with_bias):
    q, s, w_ref = make_weight(n, k, m + n + k, dev)
    x = torch.randn(m, k, generator=seeded(3)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(4)) * 0.02).to(torch.bfloat16).to(dev) if with_bias else None
    check_close(int8_row_linear(x, q, s, (n, k), b), oracle_linear(x, w_ref, b))


@pytest.mark.parametrize("k", [128, 320, 2048])
def test_tiled_bits_beside_another_kernel(dev, k):
    # K/64 = 2 (mod 3): the K blocks after the unrolled loop of three must wait for all their loads. Run
    # while an elementwise kernel streams 256 MB on another stream, the tiled int8 GEMM gives the bits of
    # the same launch alone.
    n = 1024
    q, s, _ = make_weight(n, k, 31, dev)
    x = torch.randn(16384, k, generator=seeded(32)).to(torch.bfloat16).to(dev)
    ref = int8_row_linear(x, q, s, (n, k))
    big = torch.randn(64 << 20, device=dev)
    other = torch.cuda.Stream(dev)
    torch.cuda.synchronize()
    outs = []
    for _ in range(4):
        with torch.cuda.stream(other):
            big.mul_(1.0)
        outs.append(int8_row_linear(x, q, s, (n, k)))
    torch.cuda.synchronize()
    assert all(torch.equal(y, ref) for y in outs)


def test_tiled_split_tail(dev):
    # M = 16640, N = 1024, K = 2048: 260 tiles of 256 x 256; on 256 CUs the last row slab's 4 tiles run as 8
    # K ranges each, summed in K order by a second kernel. The whole tiles equal a launch of their rows alone
    # bit for bit, the split ones agree with an unsplit launch to the order of the fp32 sums, and sampled rows
    # of both match the oracle.
    m, n, k = 16640, 1024, 2048
    q, s, w_ref = make_weight(n, k, 41, dev)
    x = torch.randn(m, k, generator=seeded(42)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(43)) * 0.02).to(torch.bfloat16).to(dev)
    y = int8_row_linear(x, q, s, (n, k), b)
    assert torch.equal(int8_row_linear(x, q, s, (n, k), b), y)
    assert torch.equal(y[:16384], int8_row_linear(x[:16384], q, s, (n, k), b))
    alone = int8_row_linear(x[16384:], q, s, (n, k), b).double()
    assert ((y[16384:].double() - alone).norm() / alone.norm()).item() < 1e-4
    rows = torch.cat([torch.randint(0, 16384, (64,), generator=seeded(44)), torch.arange(16384, m, 4)])
    check_close(y[rows], oracle_linear(x[rows], w_ref, b))


def test_tiled_operand_is_the_reference_decode_bit_for_bit(dev):
    n, k, m = 320, 640, 96
    q, s, w_ref = make_weight(n, k, 7, dev)
    ks = torch.randint(0, k, (m,), generator=seeded(8))
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    x[torch.arange(m), ks] = 1.0
    y = int8_row_linear(x.to(dev), q, s, (n, k)).float().cpu()
    assert torch.equal(y, w_ref[:, ks].t())


def test_skinny_operand_within_one_rounding(dev):
    n, k, m = 192, 3072, 16
    q, s, w_ref = make_weight(n, k, 9, dev)
    ks = torch.randint(0, k, (m,), generator=seeded(10))
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    x[torch.arange(m), ks] = 1.0
    y = int8_row_linear(x.to(dev), q, s, (n, k)).float().cpu()
    ref = w_ref[:, ks].t()
    assert ((y - ref).abs() <= 2.0 ** -7 * ref.abs()).all()


def test_strided_input_and_deterministic(dev):
    n, k = 256, 192
    q, s, w_ref = make_weight(n, k, 11, dev)
    base = torch.randn(2, 70, k + 64, generator=seeded(12)).to(torch.bfloat16).to(dev)
    x = base[:, 3:, 32:32 + k]
    y = int8_row_linear(x, q, s, (n, k))
    assert torch.equal(y, int8_row_linear(x, q, s, (n, k)))
    check_close(y.reshape(-1, n), oracle_linear(x.reshape(-1, k), w_ref))


def test_unsupported_shape_falls_back_to_decode_and_library_gemm(dev):
    n, k = 96, 96  # K % 64 != 0
    q, s, w_ref = make_weight(n, k, 13, dev)
    for m in (8, 40):
        x = torch.randn(m, k, generator=seeded(14)).to(torch.bfloat16).to(dev)
        with pytest.raises(_lib.Unsupported):
            _lib.call("selas_int8_row_linear", x.data_ptr(), m, k, k, q.data_ptr(), s.data_ptr(), n, None,
                      torch.empty(m, n, dtype=torch.bfloat16, device=dev).data_ptr(), n, _lib.BF16, None, 0,
                      _lib.stream(dev))
        check_close(int8_row_linear(x, q, s, (n, k)), oracle_linear(x, w_ref))


def test_batched_and_gelu_equal_one_by_one(dev):
    from selas_amd.kernels import Kernels

    shapes = [(300, 512, 3072), (64, 256, 640), (512, 768, 1024), (100, 256, 64), (1000, 96, 128)]
    probs, refs = [], []
    for i, (m, n, k) in enumerate(shapes):
        q, s, w_ref = make_weight(n, k, 70 + i, dev)
        x = torch.randn(m, k, generator=seeded(80 + i)).to(torch.bfloat16).to(dev)
        b = (torch.randn(n, generator=seeded(90 + i)) * 0.02).to(torch.bfloat16).to(dev) if i % 2 else None
        probs.append((x, q, s, (n, k), b))
        refs.append(w_ref)
    ys = int8_row_linear_batched(probs)
    for prob, w_ref, y in zip(probs, refs, ys):
        assert torch.equal(y, int8_row_linear(*prob))
        check_close(y, oracle_linear(prob[0], w_ref, prob[4]))
    # GELU on the last 256 columns of the first three (fused epilogue), into strided outputs.
    gp = []
    for x, q, s, shape, b in probs[:3]:
        out = torch.zeros(x.shape[0], 256 + 32, dtype=torch.bfloat16, device=dev)[:, 16:16 + 256]
        gp.append((x, q, s, shape, b, 256, out))
    for (x, q, s, shape, b, gc, out), (y, g) in zip(gp, int8_row_linear_gelu(gp)):
        full = int8_row_linear(x, q, s, shape, b)
        n = shape[0]
        assert g.data_ptr() == out.data_ptr() and torch.equal(g, Kernels().gelu(full[:, n - gc:]))
        assert (y is None) == (gc == n) and (y is None or torch.equal(y, full[:, :n - gc]))


def test_unit_view_dispatches_int8_row(dev):
    n, k = 512, 256
    w = torch.randn(n, k, generator=seeded(17)) * 0.02
    e = codecs.encode_int8_row("lin.weight", w.to(dev))
    b = codecs.encode_raw("lin.bias", (torch.randn(n, generator=seeded(18)) * 0.02).to(dev), torch.bfloat16)
    view = UnitView({"lin.weight": e, "lin.bias": b}, torch.bfloat16)
    w_ref = view.get("lin.weight").float().cpu()  # the decode kernel, bit-exact with the oracle
    assert np.array_equal(bits(view.get("lin.weight")),
                          oi8.decode(e.parts["q"].cpu().numpy(), e.parts["scale"].cpu().numpy(), oi8.BF16))
    for m in (20, 80):
        x = torch.randn(1, m, k, generator=seeded(19)).to(torch.bfloat16).to(dev)
        y = view.linear(x, "lin")
        check_close(y.reshape(-1, n), oracle_linear(x.reshape(-1, k), w_ref, b.parts["data"]))
        (y2,) = view.linear_many([(x, "lin")])
        assert torch.equal(y, y2)


def test_grouped_skinny_equals_one_by_one(dev):
    from selas_amd.linear import int8_row_linear_grouped

    shapes = [(3072 * 6, 3072), (192, 3072), (64, 3072), (100, 3072), (3072 * 3, 3072)]
    ws, refs = [], []
    for i, (n, k) in enumerate(shapes):
        q, s, w_ref = make_weight(n, k, 40 + i, dev)
        b = (torch.randn(n, generator=seeded(50 + i)) * 0.02).to(torch.bfloat16).to(dev) if i % 2 == 0 else None
        ws.append((q, s, (n, k), b))
        refs.append(w_ref)
    for m in (1, 28, 32):
        x = torch.nn.functional.silu(torch.randn(m, 1, 3072, generator=seeded(m))).to(torch.bfloat16).to(dev)
        ys = int8_row_linear_grouped(x, ws)
        for w, w_ref, y in zip(ws, refs, ys):
            alone = int8_row_linear(x, *w)
            assert y.shape == alone.shape == (m, 1, w[2][0])
            assert torch.equal(y, alone)  # same bits as the per-linear call
            check_close(y.reshape(m, -1), oracle_linear(x.reshape(m, -1), w_ref, w[3]))


@pytest.mark.parametrize("k", [1024, 2048])
def test_streaming_skinny_other_k(dev, k):
    n, m = 416, 20
    q, s, w_ref = make_weight(n, k, k, dev)
    x = torch.randn(m, k, generator=seeded(k + 1)).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, generator=seeded(k + 2)) * 0.02).to(torch.bfloat16).to(dev)
    check_close(int8_row_linear(x, q, s, (n, k), b), oracle_linear(x, w_ref, b))


@pytest.mark.parametrize("k", [1024, 2048, 3072])
def test_streaming_skinny_every_m_with_strided_x(dev, k):
    # x goes through LDS as in the NF4 kernel: every M from 1 to 32, x a column slice of a wider buffer.
    n = 160
    q, s, w_ref = make_weight(n, k, 9 + k, dev)
    wide = torch.randn(32, k + 192, generator=seeded(k + 5)).to(torch.bfloat16).to(dev)
    for m in range(1, 33):
        x = wide[:m, 64:64 + k]
        y = int8_row_linear(x, q, s, (n, k))
        check_close(y, oracle_linear(x, w_ref))
        assert torch.equal(y, int8_row_linear(x.contiguous(), q, s, (n, k)))


def test_full_size_single_linear(dev):
    # The 1536-token linear (W 12288 x 3072 ~ N(0, 0.02) seed 0, X 1536 x 3072 seed 1) with int8_row
    # weights: rows sampled against the oracle.
    n, k, m = 12288, 3072, 1536
    w = torch.randn(n, k, generator=seeded(0)) * 0.02
    e = codecs.encode_int8_row("w", w.to(dev))
    x = torch.randn(m, k, generator=seeded(1)).to(torch.bfloat16).to(dev)
    y = int8_row_linear(x, e.parts["q"], e.parts["scale"], (n, k))
    w_ref = torch.from_numpy(onf4.bf16_to_f32(oi8.decode(e.parts["q"].cpu().numpy(), e.parts["scale"].cpu().numpy(),
                                                        oi8.BF16))).view(n, k)
    rows = torch.randint(0, m, (64,), generator=seeded(2))
    check_close(y[rows], oracle_linear(x[rows], w_ref))
    assert torch.isfinite(y).all()
