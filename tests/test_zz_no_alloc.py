"""selas_nf4_linear_grouped_static, the grouped skinny linear that allocates nothing (descriptors in host
memory, staged in the library's own per-stream tables), against selas_nf4_linear_grouped (descriptors in a
caller-allocated device array), through the C ABI: bit for bit, on two calls in a row, the second with
fewer weights, fewer rows and another K; on two streams at once; past one copy batch of descriptors (76 and
1023 weights); and a stream beyond the tables is refused."""

from __future__ import annotations

import ctypes

import pytest
import torch

from selas_amd import _lib, codecs
from selas_amd.linear import GroupedPlan

from .conftest import seeded

pytestmark = pytest.mark.gpu


def weights(ns, k, seed, dev, with_bias):
    g = seeded(seed)
    out = []
    for i, n in enumerate(ns):
        e = codecs.encode_nf4("w", (torch.randn(n, k, generator=g) * 0.02).to(dev))
        b = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16).to(dev) if with_bias(i) else None
        out.append((e, b))
    return out


def run_static(x, ws, dev):
    m, k = x.shape
    ys = [torch.full((m, e.shape[0]), float("nan"), dtype=torch.bfloat16, device=dev) for e, _ in ws]
    static_call(x, ws, ys, dev)
    return ys


def static_call(x, ws, ys, dev):
    m, k = x.shape
    arr = (_lib.GemvDesc * len(ws))()
    for i, ((e, b), y) in enumerate(zip(ws, ys)):
        arr[i] = _lib.GemvDesc(e.parts["packed"].data_ptr(), e.parts["absmax"].data_ptr(), _lib.ptr(b), y.data_ptr(),
                               e.shape[0], e.shape[0])
    with torch.cuda.device(dev):
        _lib.call("selas_nf4_linear_grouped_static", x.data_ptr(), m, k, x.stride(0), ctypes.addressof(arr), len(ws),
                  64, _lib.code_array(codecs.NF4_CODE), _lib.BF16, _lib.stream(dev))
    del arr  # host descriptors are read during the call only


def run_device_descs(x, ws, dev):
    plan = GroupedPlan([(e.parts["packed"], e.parts["absmax"], 64, codecs.NF4_CODE, e.shape, b) for e, b in ws],
                       x.shape[0], dev)
    assert plan.supported
    return [y.clone() for y in plan.run(x)]


def test_static_grouped_equals_grouped_on_two_calls(dev):
    k1, n1 = 3072, [18432, 9216, 3072, 256, 9216, 32, 6144, 9216, 512, 18432, 96, 4096]
    w1 = weights(n1, k1, 61, dev, lambda i: i % 3 != 1)
    x1 = torch.nn.functional.silu(torch.randn(28, k1, generator=seeded(62))).to(torch.bfloat16).to(dev)
    a1 = run_static(x1, w1, dev)
    torch.cuda.synchronize(dev)
    b1 = run_device_descs(x1, w1, dev)
    for a, b in zip(a1, b1):
        assert torch.equal(a, b)
    # second call: fewer weights, fewer rows, another K; the table keeps the first call's entries past these
    k2, n2 = 2048, [640, 9216, 64, 3072, 160]
    w2 = weights(n2, k2, 63, dev, lambda i: i != 2)
    x2 = torch.randn(9, k2, generator=seeded(64)).to(torch.bfloat16).to(dev)
    a2 = run_static(x2, w2, dev)
    b2 = run_device_descs(x2, w2, dev)
    for a, b in zip(a2, b2):
        assert torch.equal(a, b)
    # and each equals the single-weight entry point
    for (e, b), y in zip(w2, a2):
        one = torch.empty_like(y)
        with torch.cuda.device(dev):
            _lib.call("selas_nf4_linear", x2.data_ptr(), 9, k2, k2, e.parts["packed"].data_ptr(),
                      e.parts["absmax"].data_ptr(), 64, _lib.code_array(codecs.NF4_CODE), e.shape[0], _lib.ptr(b),
                      one.data_ptr(), e.shape[0], _lib.BF16, None, 0, _lib.stream(dev))
        assert torch.equal(one, y)


def test_static_grouped_rejects_too_many_weights_and_bad_shapes(dev):
    x = torch.zeros(4, 3072, dtype=torch.bfloat16, device=dev)
    arr = (_lib.GemvDesc * 1)()
    code = _lib.code_array(codecs.NF4_CODE)
    with pytest.raises(ValueError, match="at most 1023"):
        _lib.call("selas_nf4_linear_grouped_static", x.data_ptr(), 4, 3072, 3072, ctypes.addressof(arr),
                  _lib.STATIC_MAX_WEIGHTS + 1, 64, code, _lib.BF16, _lib.stream(dev))
    with pytest.raises(ValueError):  # descriptor with n = 0
        _lib.call("selas_nf4_linear_grouped_static", x.data_ptr(), 4, 3072, 3072, ctypes.addressof(arr), 1, 64, code,
                  _lib.BF16, _lib.stream(dev))
    with pytest.raises(_lib.Unsupported):  # M > 32
        _lib.call("selas_nf4_linear_grouped_static", x.data_ptr(), 33, 3072, 3072, ctypes.addressof(arr), 1, 64, code,
                  _lib.BF16, _lib.stream(dev))


class _Slice:
    """Weight i of one encoded [count * n, k] tensor: its rows' codes and scales, in place."""

    def __init__(self, e, i, n, k):
        self.shape = (n, k)
        self.parts = {"packed": e.parts["packed"][i * n * k // 2:(i + 1) * n * k // 2],
                      "absmax": e.parts["absmax"][i * n * k // 64:(i + 1) * n * k // 64]}


def many_weights(count, n, k, seed, dev):
    g = seeded(seed)
    e = codecs.encode_nf4("w", (torch.randn(count * n, k, generator=g) * 0.02).to(dev))
    bias = (torch.randn(count * n, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    return [(_Slice(e, i, n, k), bias[i * n:(i + 1) * n] if i % 2 else None) for i in range(count)]


@pytest.mark.parametrize("count,n,k", [(76, 96, 3072), (1023, 32, 1024)])
def test_static_grouped_past_one_descriptor_batch(dev, count, n, k):
    # Descriptors reach the table in batches of 64 per copy launch: 76 weights (the FLUX modulation count)
    # take two batches, 1023 (the maximum) sixteen.
    ws = many_weights(count, n, k, 70 + count, dev)
    x = torch.nn.functional.silu(torch.randn(28, k, generator=seeded(71))).to(torch.bfloat16).to(dev)
    a = run_static(x, ws, dev)
    b = run_device_descs(x, ws, dev)
    assert len(a) == count
    for i, (ya, yb) in enumerate(zip(a, b)):
        assert torch.equal(ya, yb), i


def test_static_grouped_on_two_streams_at_once(dev):
    # Each stream stages into a table of its own: calls enqueued on two streams without a synchronisation
    # between them, with different weight counts, K and rows, give the device-descriptor path's bits.
    wa = many_weights(76, 64, 3072, 81, dev)
    wb = weights([640, 9216, 64, 3072, 160], 2048, 82, dev, lambda i: i != 2)
    xa = torch.nn.functional.silu(torch.randn(28, 3072, generator=seeded(83))).to(torch.bfloat16).to(dev)
    xb = torch.randn(9, 2048, generator=seeded(84)).to(torch.bfloat16).to(dev)
    ra, rb = run_device_descs(xa, wa, dev), run_device_descs(xb, wb, dev)
    sa, sb = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    ya = [[torch.full((28, 64), float("nan"), dtype=torch.bfloat16, device=dev) for _ in wa] for _ in range(3)]
    yb = [[torch.full((9, e.shape[0]), float("nan"), dtype=torch.bfloat16, device=dev) for e, _ in wb]
          for _ in range(3)]
    torch.cuda.synchronize(dev)
    for r in range(3):
        with torch.cuda.stream(sa):
            static_call(xa, wa, ya[r], dev)
        with torch.cuda.stream(sb):
            static_call(xb, wb, yb[r], dev)
    torch.cuda.synchronize(dev)
    for r in range(3):
        assert all(torch.equal(y, ref) for y, ref in zip(ya[r], ra))
        assert all(torch.equal(y, ref) for y, ref in zip(yb[r], rb))


def test_static_grouped_refuses_a_stream_beyond_its_tables(dev):
    # SELAS_STATIC_MAX_STREAMS tables per GPU: with the default stream's table taken by the tests above,
    # 8 more streams cannot all get one. The refused calls launch nothing; the others give the usual bits.
    ws = weights([256, 96], 1024, 91, dev, lambda i: True)
    x = torch.randn(5, 1024, generator=seeded(92)).to(torch.bfloat16).to(dev)
    run_static(x, ws, dev)  # the default stream holds a table
    ref = run_device_descs(x, ws, dev)
    streams = [torch.cuda.Stream(dev) for _ in range(_lib.STATIC_MAX_STREAMS)]
    refused = 0
    for st in streams:
        ys = [torch.full((5, e.shape[0]), float("nan"), dtype=torch.bfloat16, device=dev) for e, _ in ws]
        with torch.cuda.stream(st):
            try:
                static_call(x, ws, ys, dev)
            except _lib.Unsupported as err:
                assert "streams" in str(err)
                refused += 1
                continue
        st.synchronize()
        assert all(torch.equal(y, r) for y, r in zip(ys, ref))
    assert refused >= 1
