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
        _lib.call("selas_nf4_linear", null, 4, 64, 64, null, null, 64, _code(), 8, null, null, 8, _lib.BF16, null)
    with pytest.raises(_lib.Unsupported, match="blocksize 64"):
        x = ctypes.c_void_p(16)
        _lib.call("selas_nf4_linear", x, 4, 96, 96, x, x, 32, _code(), 8, null, x, 8, _lib.BF16, null)
    with pytest.raises(_lib.Unsupported, match="D <="):
        _lib.call("selas_mod_in", null, 1, 1, 8192, 0, 8192, null, null, 0, null, _lib.BF16, null)
    with pytest.raises(_lib.Unsupported, match="head_dim"):
        _lib.call("selas_qkv_single", null, 1, 4, 2, 256, 0, 1536, null, null, null, null, null, null, null,
                  _lib.BF16, null)
    assert lib.selas_last_error().decode()  # the message stays readable
    # empty work is a no-op that succeeds
    _lib.call("selas_nf4_dequant", null, null, 0, 64, _code(), null, _lib.BF16, null)
    _lib.call("selas_nf4_linear", null, 0, 64, 64, null, null, 64, _code(), 8, null, null, 8, _lib.BF16, null)


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
    with pytest.raises(ValueError):
        kernels._bld(torch.zeros(4, 4).t(), "x")


def test_gelu_columns_are_checked():
    # Validation before any device work: the GELU columns must start at a multiple of the 256-column tile.
    x = ctypes.c_void_p(4096)
    arr = (_lib.GemmProblem * 1)()
    arr[0] = _lib.GemmProblem(4096, 64, 64, 64, 4096, 4096, 512, None, 4096, 512, 4096, 300, 300)
    with pytest.raises(_lib.Unsupported, match="multiple of 256"):
        _lib.call("selas_nf4_linear_batched", ctypes.addressof(arr), 1, 64, _code(), _lib.BF16, None)
    arr[0].gelu_cols = 600
    with pytest.raises(ValueError, match="gelu_cols"):
        _lib.call("selas_nf4_linear_batched", ctypes.addressof(arr), 1, 64, _code(), _lib.BF16, None)
    arr[0].gelu_cols, arr[0].y2 = 256, None
    with pytest.raises(ValueError, match="y2"):
        _lib.call("selas_nf4_linear_batched", ctypes.addressof(arr), 1, 64, _code(), _lib.BF16, None)
    del x
