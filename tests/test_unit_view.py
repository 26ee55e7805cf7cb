"""UnitView built as selas's store builds it (spec + uint8 unit buffer + dtype), on the CPU: parts are
viewed in place (selas/container.py:79-82, store.py:245-263); no kernel runs here."""

from __future__ import annotations

from dataclasses import dataclass, field

import pytest
import torch

from selas_amd.linear import UnitView, part_view


@dataclass(frozen=True)
class PartSpec:
    offset: int
    nbytes: int
    dtype: str
    shape: tuple


@dataclass
class TensorSpec:
    codec: str
    shape: tuple
    meta: dict
    parts: dict = field(default_factory=dict)


@dataclass
class UnitSpec:
    tensors: dict


def test_parts_are_views_into_the_unit_buffer():
    buf = torch.zeros(4096, dtype=torch.uint8)
    scale = torch.arange(128, dtype=torch.float32)
    buf[256:256 + 512] = scale.view(torch.uint8)
    codes = torch.arange(96, dtype=torch.uint8)
    buf[1024:1024 + 96] = codes
    absmax = torch.full((3,), 0.5)
    buf[1280:1280 + 12] = absmax.view(torch.uint8)
    spec = UnitSpec({
        "norm.scale": TensorSpec("raw", (128,), {}, {"data": PartSpec(256, 512, "float32", (128,))}),
        "lin.weight": TensorSpec("nf4", (3, 64), {"blocksize": 64, "code": [0.0] * 16},
                                 {"packed": PartSpec(1024, 96, "uint8", (96,)),
                                  "absmax": PartSpec(1280, 12, "float32", (3,))}),
    })
    u = UnitView(spec, buf, torch.bfloat16)
    assert u.has("lin.weight") and u.codec("lin.weight") == "nf4" and not u.has("x")
    p = u.parts("lin.weight")
    assert torch.equal(p["packed"], codes) and torch.equal(p["absmax"], absmax)
    assert p["packed"].untyped_storage().data_ptr() == buf.untyped_storage().data_ptr()
    # raw tensors in their stored dtype come back as zero-copy views of the buffer
    got = u.get("norm.scale", torch.float32)
    assert torch.equal(got, scale) and got.data_ptr() == buf.data_ptr() + 256
    assert torch.equal(part_view(buf, spec.tensors["norm.scale"].parts["data"]), scale)
    buf[256:260] = torch.tensor([1.5], dtype=torch.float32).view(torch.uint8)
    assert got[0].item() == 1.5  # a view, not a copy


def test_unit_buffer_must_be_uint8_1d():
    spec = UnitSpec({})
    with pytest.raises(ValueError):
        UnitView(spec, torch.zeros(16, dtype=torch.float32), torch.bfloat16)
    with pytest.raises(ValueError):
        UnitView(spec, torch.zeros(4, 4, dtype=torch.uint8), torch.bfloat16)
