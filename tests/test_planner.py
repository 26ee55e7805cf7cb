"""Cost accounting with the fused linears (selas_amd.planner) against the reference planner's rules
(selas/pipeline.py:151-165, 238-245): host logic, no GPU."""

from __future__ import annotations

from types import SimpleNamespace as NS

import pytest
import torch

from selas_amd import planner as P
from selas_amd.flux import FluxConfig, unit_flops


def spec(codec, shape, meta=None, stored=None):
    return NS(codec=codec, shape=shape, meta=meta or {}, stored_dtype=stored)


def test_fused_codecs_have_no_decode_temporary():
    bf = torch.bfloat16
    assert P.decoded_bytes(spec("nf4", (21504, 3072), {"blocksize": 64}), bf) == 0
    assert P.decoded_bytes(spec("int8_row", (3072, 15360)), bf) == 0
    # outside the fused kernels the weight is decoded, as in the reference
    assert P.decoded_bytes(spec("nf4", (96, 96), {"blocksize": 32}), bf) == 96 * 96 * 2
    assert P.decoded_bytes(spec("nf4", (128, 256), {"blocksize": 64}), torch.float16) == 128 * 256 * 2
    assert P.decoded_bytes(spec("int8_row", (64, 100)), bf) == 64 * 100 * 2
    # raw: a view when stored in the compute dtype, a cast copy otherwise
    assert P.decoded_bytes(spec("raw", (3072, 3072), stored="bfloat16"), bf) == 0
    assert P.decoded_bytes(spec("raw", (3072, 3072), stored="float8_e4m3fn"), bf) == 3072 * 3072 * 2
    # 1-D tensors (biases, norm scales) never count
    assert P.decoded_bytes(spec("raw", (3072,), stored="float32"), bf) == 0


def test_decode_temp_bytes_is_the_largest_remaining_temporary():
    units = [{"a": spec("nf4", (21504, 3072), {"blocksize": 64}), "b": spec("raw", (64, 64), stored="float32")},
             {"c": spec("int8_row", (3072, 15360)), "d": spec("nf4", (96, 96), {"blocksize": 32})}]
    assert P.decode_temp_bytes(units, torch.bfloat16) == 96 * 96 * 2
    assert P.decode_temp_bytes([units[0]], torch.bfloat16) == 64 * 64 * 2
    assert P.decode_temp_bytes([{"a": units[0]["a"]}], torch.bfloat16) == 0


def test_estimate_follows_the_reference_formula():
    cfg = FluxConfig()
    hw = P.HwProfile(matmul_flops=1e15, attn_flops=5e14, mem_bw=4e12, dequant_bw=1e12)
    fused = {"linear1.weight": spec("nf4", (21504, 3072), {"blocksize": 64}),
             "linear2.weight": spec("nf4", (3072, 15360), {"blocksize": 64})}
    lin, att = unit_flops("single", cfg, 4096, 512, 1)
    base = lin / 1e15 + att / 5e14 + 4608 * 3072 * 100 / 4e12
    assert P.estimate_seconds("single", cfg, 4096, 512, 1, fused, hw) == pytest.approx(base)
    decoded = {k: spec("raw", v.shape, stored="float16") for k, v in fused.items()}
    extra = (21504 * 3072 + 3072 * 15360) * 2 / 1e12
    assert P.estimate_seconds("single", cfg, 4096, 512, 1, decoded, hw) == pytest.approx(base + extra)


def test_profile_fields_match_the_reference():
    names = {"h2d_bw", "disk_bw", "matmul_flops", "attn_flops", "mem_bw", "dequant_bw", "measured"}
    assert set(P.HwProfile.__dataclass_fields__) == names
