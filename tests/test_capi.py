"""The C ABI without a GPU: the library loads, exports every declared symbol, and rejects bad
arguments before touching the device. Also the host-side logic of the Python wrappers."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from selas_amd import _lib, codecs, kernels

HEADER = Path(__file__).resolve().parent.parent / "include" / "selas_amd.h"


def declared_symbols() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(selas_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert "selas_nf4_linear" in names and len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert set(_lib.SIGNATURES) | {"selas_last_error", "selas_abi_version"} == set(names)
    assert lib.selas_abi_version() == _lib.ABI_VERSION


def _code():
    return _lib.code_array(codecs.NF4_CODE)


def test_invalid_arguments_are_reported_without_a_device_call():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    with pytest.raises(ValueError, match="blocksize"):
        _lib.call("selas_nf4_dequant", null, null, 64, 3, _code(), null, _lib.BF16, null)
    with pytest.raises(ValueError, match="dtype"):
        _lib.call("selas_nf4_dequant", null, null, 64, 64, _code(), null, 7, null)
    with pytest.raises(ValueError, match="divisible"):
        _lib.call("selas_nf4_encode", null, 100, 64, _code(), null, null, null)
    with pytest.raises(ValueError, match="null"):
        _lib.call("selas_nf4_linear", null, 4, 64, 64, null, null, 64, _code(), 8, null, null, 8, _lib.BF16, null, 0,
                  null)
    with pytest.raises(_lib.Unsupported, match="blocksize 64"):
        x = ctypes.c_void_p(16)
        _lib.call("selas_nf4_linear", x, 4, 96, 96, x, x, 32, _code(), 8, null, x, 8, _lib.BF16, null, 0, null)
    with pytest.raises(_lib.Unsupported, match="D <="):
        _lib.call("selas_mod_in", null, 1, 1, 8192, 0, 8192, null, null, 0, null, _lib.BF16, null)
    with pytest.raises(_lib.Unsupported, match="head_dim"):
        _lib.call("selas_qkv_single", null, 1, 4, 2, 256, 0, 1536, null, null, null, null, null, null, null,
                  _lib.BF16, null)
    assert lib.selas_last_error().decode()  # the message stays readable
    # empty work is a no-op that succeeds
    _lib.call("selas_nf4_dequant", null, null, 0, 64, _code(), null, _lib.BF16, null)
    _lib.call("selas_nf4_linear", null, 0, 64, 64, null, null, 64, _code(), 8, null, null, 8, _lib.BF16, null, 0,
              null)


def test_python_wrappers_validate_like_the_reference():
    with pytest.raises(ValueError, match="divisible"):
        codecs.encode_nf4("w", torch.zeros(100), 64)
    with pytest.raises(NotImplementedError, match="partial"):
        codecs.nf4_import("w", torch.zeros(32, dtype=torch.uint8), torch.ones(2), (10, 10), 64, codecs.NF4_CODE)
    with pytest.raises(ValueError):
        codecs.nf4_import("w", torch.zeros(32, dtype=torch.uint8), torch.ones(2), (8, 16), 64, codecs.NF4_CODE)
    e = codecs.nf4_import("w", torch.zeros(64, 1, dtype=torch.uint8), torch.ones(2), (8, 16), 64, codecs.NF4_CODE)
    assert e.parts["packed"].shape == (64,) and e.parts["absmax"].dtype == torch.float32
    with pytest.raises(ValueError, match="unknown codec"):
        codecs.decode("bogus", {}, {}, (1,), torch.float32)
    with pytest.raises(ValueError, match="GPU"):
        codecs.nf4_dequant(torch.zeros(32, dtype=torch.uint8), torch.ones(1), 64, codecs.NF4_CODE, (64,),
                           torch.bfloat16)
    raw = codecs.encode_raw("b", torch.arange(6.0).view(2, 3), torch.float32)
    assert codecs.decode("raw", raw.parts, raw.meta, raw.shape, torch.float32).data_ptr() == raw.parts["data"].data_ptr()
    assert codecs.decoded_is_view("raw", "bfloat16", torch.bfloat16) and not codecs.decoded_is_view("nf4", None, torch.float32)


def test_segment_stride_helpers():
    x = torch.zeros(2, 5, 8)
    assert kernels._bld(x, "x") == (2, 5, 8, 40, 8)
    assert kernels._bld(x[:, 1:], "x") == (2, 4, 8, 40, 8)
    mod = torch.zeros(2, 24).unsqueeze(1).chunk(3, dim=-1)[1]  # [2, 1, 8] view, batch stride 24
    v, sb = kernels._vec(mod, 2, 8, "m")
    assert sb == 24 and v.data_ptr() == mod.data_ptr()
    v, sb = kernels._vec(torch.zeros(1, 1, 8), 2, 8, "m")
    assert sb == 0
    h = torch.zeros(2, 3, 21)
    assert kernels.Kernels._rows2(h[..., 9:], "h") == (6, 12, 21)
    with pytest.raises(_lib.Unsupported):  # the eager segment takes such layouts
        kernels._bld(torch.zeros(4, 4).t(), "x")


def test_gelu_columns_are_checked():
    # Validation before any device work: the GELU columns must start at a multiple of the 256-column tile.
    x = ctypes.c_void_p(4096)
    arr = (_lib.GemmProblem * 1)()
    arr[0] = _lib.GemmProblem(4096, 64, 64, 64, 4096, 4096, 512, None, 4096, 512, 4096, 300, 300)
    with pytest.raises(_lib.Unsupported, match="multiple of 256"):
        _lib.call("selas_nf4_linear_batched", ctypes.addressof(arr), 1, 64, _code(), _lib.BF16, None, 0, None)
    arr[0].gelu_cols = 600
    with pytest.raises(ValueError, match="gelu_cols"):
        _lib.call("selas_nf4_linear_batched", ctypes.addressof(arr), 1, 64, _code(), _lib.BF16, None, 0, None)
    arr[0].gelu_cols, arr[0].y2 = 256, None
    with pytest.raises(ValueError, match="y2"):
        _lib.call("selas_nf4_linear_batched", ctypes.addressof(arr), 1, 64, _code(), _lib.BF16, None, 0, None)
    del x


def _ws_query(shapes, codec=_lib.CODEC_NF4):
    arr = (_lib.GemmProblem * max(len(shapes), 1))()
    for i, (m, k, n) in enumerate(shapes):
        arr[i].M, arr[i].K, arr[i].N = m, k, n
    out = ctypes.c_int64(-1)
    _lib.call("selas_linear_workspace_bytes", ctypes.addressof(arr), len(shapes), codec, ctypes.byref(out))
    return out.value


def test_split_workspace_is_sized_from_shapes_only():
    # The split plan is host logic over (M, K, N) and the CU count (256 on MI355X; the fallback when no GPU
    # answers). 4 x 1536 tokens x 3072 x 15360 (the 512^2 batch-4 linear2): 24 x 12 = 288 tiles of 256 x 256,
    # a last round of 32 run as 8 K ranges -> 32 x 8 x 256 KiB. 16640 x 1024 x 2048: 4 tiles past one round,
    # 8 ranges each. The 1024^2 block linears, a skinny M and the 1536-token linear (K 3072, below the split's
    # margin) need none; int8_row plans its splits the same way.
    kib = 1024
    assert _ws_query([(6144, 15360, 3072)]) == 32 * 8 * 256 * kib
    assert _ws_query([(6144, 15360, 3072)], _lib.CODEC_INT8_ROW) == 32 * 8 * 256 * kib
    assert _ws_query([(16640, 2048, 1024)]) == 4 * 8 * 256 * kib
    assert _ws_query([(4096, 12288, 3072), (2048, 12288, 3072)]) > 0  # the 512^2 batch-4 mlp.2 pair
    for shapes in ([(4608, 3072, 21504)], [(4608, 15360, 3072)], [(1536, 3072, 12288)], [(28, 3072, 18432)],
                   [(0, 3072, 3072)], [], [(6144, 15360, 3072), (8, 15360, 3072)]):
        assert _ws_query(shapes) == 0, shapes
    assert _ws_query([(6144, 15360, 3072)]) == _ws_query([(6144, 15360, 3072)])  # no state between calls
    with pytest.raises(ValueError, match="codec"):
        _ws_query([(64, 64, 64)], codec=7)
    with pytest.raises(ValueError, match="count"):
        _ws_query([(64, 64, 64)] * 5)


def test_split_launch_without_its_workspace_is_refused_before_any_device_call():
    # A split shape with no (or too small, or misaligned) workspace is an argument error, never an unsplit launch.
    x = ctypes.c_void_p(1 << 20)
    m, k, n = 16640, 2048, 1024
    need = 4 * 8 * 256 * 1024
    for ws, nbytes in ((None, 0), (x, need - 1), (ctypes.c_void_p((1 << 20) + 8), need)):
        with pytest.raises(ValueError, match="workspace of 8388608 bytes"):
            _lib.call("selas_nf4_linear", x, m, k, k, x, x, 64, _code(), n, None, x, n, _lib.BF16, ws, nbytes, None)
        with pytest.raises(ValueError, match="workspace"):
            _lib.call("selas_int8_row_linear", x, m, k, k, x, x, n, None, x, n, _lib.BF16, ws, nbytes, None)
        arr = (_lib.GemmProblem * 1)()
        arr[0] = _lib.GemmProblem(x.value, m, k, k, x.value, x.value, n, None, x.value, n)
        with pytest.raises(ValueError, match="workspace"):
            _lib.call("selas_nf4_linear_batched", ctypes.addressof(arr), 1, 64, _code(), _lib.BF16, ws, nbytes, None)


def test_grouped_skinny_refuses_an_x_of_4_gib_before_any_device_call():
    # The streaming kernels address x through a 32-bit buffer range: (M - 1) * ldx + K elements must stay
    # under 4 GiB. 32 rows at a row stride of 2^27 elements span 8.3 GB.
    x = ctypes.c_void_p(1 << 20)
    descs = (_lib.GemvDesc * 1)()
    descs[0] = _lib.GemvDesc(x.value, x.value, None, x.value, 96, 96)
    m, k, ldx = 32, 3072, 1 << 27
    with pytest.raises(_lib.Unsupported, match="4 GiB"):
        _lib.call("selas_nf4_linear_grouped", x, m, k, ldx, x, 1, 96, 64, _code(), _lib.BF16, None)
    with pytest.raises(_lib.Unsupported, match="4 GiB"):
        _lib.call("selas_int8_row_linear_grouped", x, m, k, ldx, x, 1, 96, _lib.BF16, None)
    with pytest.raises(_lib.Unsupported, match="4 GiB"):
        _lib.call("selas_nf4_linear_grouped_static", x, m, k, ldx, ctypes.addressof(descs), 1, 64, _code(),
                  _lib.BF16, None)


def test_eager_segments_are_the_reference_math_and_stay_off_the_cpu():
    # The eager fallback of Kernels is the segment math of selas (flux.py:117-147, 164-200); on the CPU it
    # equals the oracle's restatement (same torch ops in the same order: bit for bit), but Kernels itself
    # refuses CPU tensors, fused or eager.
    from oracle import segments as S

    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 7, 64, generator=g)
    y = torch.randn(2, 7, 64, generator=g).to(torch.bfloat16)
    sh, sc, gt = (torch.randn(2, 1, 64, generator=g) * 0.1 for _ in range(3))
    E = kernels.EAGER_SEGMENTS
    assert torch.allclose(E["mod_in"](x, sh, sc, torch.float32), S.mod_in(x, sh, sc, torch.float32), atol=1e-5)
    assert torch.equal(E["gated_add"](x, gt, y, True), S.gated_add(x, gt, y, True))
    qkv = torch.randn(1, 6, 3 * 2 * 32, generator=g).to(torch.bfloat16)
    qs, ks = torch.ones(32) + 0.1, torch.ones(32) - 0.1
    cos, sin = S.rope_tables(torch.arange(18.0).view(6, 3), (8, 12, 12), 10000.0)
    for a, b in zip(E["qkv_single"](qkv, qs, ks, cos, sin, 2, torch.bfloat16),
                    S.qkv_single(qkv, qs, ks, cos, sin, 2, torch.bfloat16)):
        assert torch.equal(a, b)
    tq = torch.randn(1, 3, 3 * 2 * 32, generator=g).to(torch.bfloat16)
    cos9, sin9 = S.rope_tables(torch.arange(27.0).view(9, 3), (8, 12, 12), 10000.0)
    for a, b in zip(E["qkv_double"](tq, qkv, qs, ks, ks, qs, cos9, sin9, 2, torch.bfloat16),
                    S.qkv_double(tq, qkv, qs, ks, ks, qs, cos9, sin9, 2, torch.bfloat16)):
        assert torch.equal(a, b)
    h = torch.randn(3, 40, generator=g)
    assert torch.allclose(E["gelu"](h), S.gelu(h), atol=1e-6)
    with pytest.raises(ValueError, match="GPU"):
        kernels.Kernels().mod_in(x.to(torch.bfloat16), sh, sc, torch.bfloat16)  # would be eager, but on the CPU
    with pytest.raises(ValueError, match="GPU"):
        kernels.Kernels().attn_mlp(x, x)
