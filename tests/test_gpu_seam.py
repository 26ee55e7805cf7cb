"""The drop-in seam as selas's engine uses it, on the GPU.

1. Units laid out as selas's container lays them out (selas/container.py:1-30, 213-258): one 4 KiB-aligned
   uint8 device buffer per unit, every tensor part at a 256-byte-aligned offset inside it, read through
   uint8 -> dtype views (part_view, container.py:79-82). ``UnitView(spec, buf, dtype)`` is built the way
   selas's store builds its UnitView (store.py:245-251) and its ``linear`` (the patched
   UnitView.linear, store.py:289-293) runs NF4 and int8_row weights from those views against the oracle.
2. NF4 weights in the bitsandbytes / Forge serialization (packed codes as uint8 [n, 1], fp32 absmax or
   double-quantized uint8 absmax with nested statistics, a quant_map and a JSON quant state:
   tests/test_convert.py:17-26 of the reference) imported as SourceView.encoded_nf4 does
   (selas/sources.py:114-127) through ``nf4_import`` (codecs.py:122-145), then decoded on the GPU
   bit-exactly and used by the fused linear.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field

import numpy as np
import pytest
import torch

from oracle import int8_row as oi8
from oracle import nf4 as onf4
from selas_amd import codecs
from selas_amd.linear import UnitView, nf4_linear, part_view

from .conftest import seeded

pytestmark = pytest.mark.gpu

UNIT_ALIGN, PART_ALIGN = 4096, 256


@dataclass(frozen=True)
class PartSpec:
    offset: int
    nbytes: int
    dtype: str
    shape: tuple


@dataclass
class TensorSpec:
    name: str
    codec: str
    shape: tuple
    meta: dict
    parts: dict = field(default_factory=dict)


@dataclass
class UnitSpec:
    name: str
    tensors: dict
    nbytes: int = 0


def align(n, a):
    return (n + a - 1) // a * a


def lay_out(name, encoded: dict, dev):
    """A unit's tensors (name -> EncodedTensor with CPU parts) packed back to back into one uint8 device
    buffer, each part at a 256-byte-aligned offset; the buffer is a 4 KiB-aligned allocation whose size is
    padded to 4 KiB (the container's unit layout)."""
    off, specs, blobs = 0, {}, []
    for tname, e in encoded.items():
        ts = TensorSpec(tname, e.codec, tuple(e.shape), dict(e.meta))
        for pname, t in e.parts.items():
            raw = t.contiguous().view(-1).view(torch.uint8)
            off = align(off, PART_ALIGN)
            ts.parts[pname] = PartSpec(off, raw.numel(), str(t.dtype).removeprefix("torch."), tuple(t.shape))
            blobs.append((off, raw))
            off += raw.numel()
        specs[tname] = ts
    size = align(off, UNIT_ALIGN)
    host = torch.zeros(size, dtype=torch.uint8)
    for o, raw in blobs:
        host[o:o + raw.numel()] = raw
    buf = torch.empty(size + UNIT_ALIGN, dtype=torch.uint8, device=dev)
    start = (-buf.data_ptr()) % UNIT_ALIGN
    buf = buf[start:start + size]
    buf.copy_(host)
    assert buf.data_ptr() % UNIT_ALIGN == 0
    return UnitSpec(name, specs, size), buf


def oracle_nf4(packed: np.ndarray, absmax: np.ndarray, shape, code=onf4.NF4_CODE):
    bits = onf4.c_decode(packed.reshape(-1), absmax.reshape(-1).astype(np.float32), 64, code, out=onf4.BF16)
    return torch.from_numpy(onf4.bf16_to_f32(bits)).view(*shape)


def check(y, ref):
    y = y.double().cpu()
    assert (y - ref).abs().max() <= 1e-2 * ref.abs().max()
    assert ((y - ref).norm() / ref.norm()).item() <= 4e-3


def test_unit_view_over_a_selas_unit_buffer(dev):
    g = seeded(51)
    w_nf4 = torch.randn(768, 640, generator=g) * 0.02
    w_i8 = torch.randn(512, 768, generator=g) * 0.02
    b1 = (torch.randn(768, generator=g) * 0.02).to(torch.bfloat16)
    scale = 1 + 0.02 * torch.randn(128, generator=g)
    e1 = codecs.encode_nf4("lin1.weight", w_nf4)  # CPU in, CPU parts out, as selas's convert step
    e2 = codecs.encode_int8_row("lin2.weight", w_i8)
    enc = {"lin1.weight": e1, "lin1.bias": codecs.encode_raw("lin1.bias", b1),
           "lin2.weight": e2, "norm.scale": codecs.encode_raw("norm.scale", scale)}
    spec, buf = lay_out("double.0", enc, dev)
    for ts in spec.tensors.values():
        for ps in ts.parts.values():
            assert ps.offset % PART_ALIGN == 0
    u = UnitView(spec, buf, torch.bfloat16)
    # parts are views into the unit buffer, not copies
    pk = u.parts("lin1.weight")["packed"]
    assert pk.untyped_storage().data_ptr() == buf.untyped_storage().data_ptr()
    assert torch.equal(part_view(buf, spec.tensors["norm.scale"].parts["data"]).cpu(), scale)
    assert u.get("norm.scale", torch.float32).data_ptr() == u.get("norm.scale", torch.float32).data_ptr()
    x = torch.randn(300, 640, generator=g).to(torch.bfloat16)
    y = u.linear(x.to(dev), "lin1")
    w1 = oracle_nf4(e1.parts["packed"].numpy(), e1.parts["absmax"].numpy(), (768, 640))
    check(y, x.double() @ w1.double().t() + b1.double())
    x2 = torch.randn(20, 768, generator=g).to(torch.bfloat16)  # skinny path over an int8_row part view
    y2 = u.linear(x2.to(dev), "lin2")
    w2 = torch.from_numpy(onf4.bf16_to_f32(oi8.decode(e2.parts["q"].numpy(), e2.parts["scale"].numpy(), oi8.BF16)))
    check(y2, x2.double() @ w2.view(512, 768).double().t())
    # decode through the unit view is the reference decode bit for bit
    assert torch.equal(u.get("lin1.weight").float().cpu(), w1)


def bnb_serialize(prefix: str, e, double_quant: bool = False) -> dict:
    """A Forge / bitsandbytes NF4 serialization of an encoded weight. With ``double_quant`` the absmax is
    stored as uint8 indices into a nested 256-entry codebook with per-256-block nested scales and an
    offset (bnb's compress_statistics)."""
    state = {"quant_type": "nf4", "blocksize": 64, "dtype": "bfloat16", "shape": list(e.shape)}
    out = {prefix: e.parts["packed"].reshape(-1, 1), prefix + ".quant_map": torch.tensor(e.meta["code"])}
    if not double_quant:
        out[prefix + ".absmax"] = e.parts["absmax"]
    else:
        a = e.parts["absmax"].double()
        offset = float(a.mean())
        c = a - offset
        nb = 256
        nested_code = torch.linspace(-1, 1, 256, dtype=torch.float64)
        blocks = c.view(-1, nb)
        nested_absmax = blocks.abs().amax(1)
        q = ((blocks / nested_absmax[:, None] + 1) * 127.5).round().clamp(0, 255).to(torch.uint8).view(-1)
        out[prefix + ".absmax"] = q
        out[prefix + ".nested_absmax"] = nested_absmax.float()
        out[prefix + ".nested_quant_map"] = nested_code.float()
        state.update({"nested_blocksize": nb, "nested_offset": offset})
    out[prefix + ".quant_state.bitsandbytes__nf4"] = torch.tensor(list(json.dumps(state).encode()), dtype=torch.uint8)
    return out


def import_bnb(sd: dict, k: str, name: str):
    """SourceView.encoded_nf4 (selas/sources.py:114-127): the JSON quant state, nested statistics
    dequantized in fp32 when present, then nf4_import of the untouched codes."""
    st = json.loads(bytes(sd[k + ".quant_state.bitsandbytes__nf4"].reshape(-1).tolist()).decode("utf-8"))
    assert st.get("quant_type", "nf4") == "nf4"
    absmax = sd[k + ".absmax"]
    if k + ".nested_absmax" in sd:
        nested_absmax = sd[k + ".nested_absmax"].float()
        nested_code = sd[k + ".nested_quant_map"].float()
        nb = int(st["nested_blocksize"])
        q = absmax.reshape(-1).to(torch.long)
        scale = nested_absmax.repeat_interleave(nb)[: q.numel()]
        absmax = nested_code[q] * scale + float(st.get("nested_offset", 0.0))
    code = sd[k + ".quant_map"].float().tolist()
    return codecs.nf4_import(name, sd[k], absmax, tuple(st["shape"]), int(st["blocksize"]), code)


@pytest.mark.parametrize("double_quant", [False, True])
def test_forge_nf4_import_decode_and_linear(dev, double_quant):
    g = seeded(52 + double_quant)
    w = torch.randn(1024, 3072, generator=g) * 0.02
    e = codecs.encode_nf4("w", w)
    sd = bnb_serialize("model.diffusion_model.double_blocks.1.img_attn.qkv.weight", e, double_quant)
    assert sd["model.diffusion_model.double_blocks.1.img_attn.qkv.weight"].shape == (1024 * 3072 // 2, 1)
    imp = import_bnb(sd, "model.diffusion_model.double_blocks.1.img_attn.qkv.weight", "img_attn.qkv.weight")
    assert imp.codec == "nf4" and imp.shape == (1024, 3072) and imp.meta["blocksize"] == 64
    assert torch.equal(imp.parts["packed"], e.parts["packed"])  # the codes are kept bit for bit
    if not double_quant:
        assert torch.equal(imp.parts["absmax"], e.parts["absmax"])
    parts = {k: v.to(dev) for k, v in imp.parts.items()}
    ref_w = oracle_nf4(imp.parts["packed"].numpy(), imp.parts["absmax"].numpy(), (1024, 3072), imp.meta["code"])
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        got = codecs.decode("nf4", parts, imp.meta, imp.shape, dt).cpu()
        if dt == torch.bfloat16:
            assert torch.equal(got.float(), ref_w)
        else:
            out = onf4.F16 if dt == torch.float16 else onf4.F32
            bits = onf4.c_decode(imp.parts["packed"].numpy(), imp.parts["absmax"].numpy(), 64, imp.meta["code"], out=out)
            want = torch.from_numpy(bits.view(np.float16) if dt == torch.float16 else bits)
            assert torch.equal(got.view(-1), want.view(-1))
    for m in (4608, 28):
        x = torch.randn(m, 3072, generator=g).to(torch.bfloat16)
        y = nf4_linear(x.to(dev), parts["packed"], parts["absmax"], 64, imp.meta["code"], imp.shape)
        rows = torch.arange(0, m, max(1, m // 160))
        check(y[rows.to(dev)], x[rows].double() @ ref_w.double().t())


def test_parts_that_do_not_match_the_shape_are_rejected(dev):
    e = codecs.encode_nf4("w", torch.randn(256, 256, generator=seeded(54)).to(dev))
    x = torch.randn(64, 256, dtype=torch.bfloat16, device=dev)
    p, a = e.parts["packed"], e.parts["absmax"]
    with pytest.raises(ValueError):
        nf4_linear(x, p[:-16], a, 64, codecs.NF4_CODE, (256, 256))  # short codes
    with pytest.raises(ValueError):
        nf4_linear(x, p, a.half(), 64, codecs.NF4_CODE, (256, 256))  # fp16 absmax
    with pytest.raises(ValueError):
        nf4_linear(x, p.view(torch.int8), a, 64, codecs.NF4_CODE, (256, 256))  # wrong code dtype
    with pytest.raises(ValueError):
        nf4_linear(x, p, a, 64, codecs.NF4_CODE, (256, 256), torch.zeros(100, dtype=torch.bfloat16, device=dev))
