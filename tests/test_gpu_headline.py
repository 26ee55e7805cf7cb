"""The headline linears at full size on the GPU against the oracle.

One FLUX single-stream block at 1024^2 (M = 4608 = 4096 image + 512 text tokens, hidden 3072): linear1
3072 -> 21504 with GELU in its epilogue writing the MLP columns into linear2's [4608, 15360] input, and
linear2 15360 -> 3072; the double block's image/text pairs (4096 / 512 tokens) in one batched launch,
including mlp.2 with K = 12288; the 1536-token linear (12288 x 3072); at 512^2 with batch 4, linear2 and
the mlp.2 pair, whose last round of tiles runs split over K. Weights N(0, 0.02) NF4 blocksize 64,
activations bf16 N(0, 1), biases bf16 N(0, 0.02).

Every output is checked on sampled rows (at least 128, all columns) against the fp64 product of x and
the oracle's decode of the same packed bytes (the reference decode, selas/codecs.py:178-199), plus the
bias: max |y - ref| <= 1e-2 * max |ref| and relative L2 <= 4e-3 (selas/store.py:289-293 is decode +
F.linear). Fused variants (the GELU epilogue, the batched launch) are also compared bit for bit with the
plain launch they replace.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nf4 as onf4
from oracle import segments as S
from selas_amd import codecs
from selas_amd.kernels import Kernels
from selas_amd.linear import nf4_linear, nf4_linear_batched, nf4_linear_gelu

from .conftest import seeded

pytestmark = pytest.mark.gpu

MAX_REL, L2_REL = 1e-2, 4e-3
D, MLP, M = 3072, 12288, 4608


def weight(n, k, seed, dev):
    """NF4 parts encoded on the GPU from seeded N(0, 0.02) values, and the oracle's decode of those bytes."""
    w = torch.randn(n, k, generator=seeded(seed)) * 0.02
    e = codecs.encode_nf4("w", w.to(dev))
    del w
    p, a = e.parts["packed"].cpu().numpy(), e.parts["absmax"].cpu().numpy()
    dec = onf4.c_decode if onf4.c_lib() else onf4.decode
    ref = torch.from_numpy(onf4.bf16_to_f32(dec(p, a, 64, out=onf4.BF16))).view(n, k)
    return e, ref


def act(m, k, seed, dev):
    return torch.randn(m, k, generator=seeded(seed)).to(torch.bfloat16).to(dev)


def bias(n, seed, dev):
    return (torch.randn(n, generator=seeded(seed)) * 0.02).to(torch.bfloat16).to(dev)


def sample_rows(m, count=160, seed=0):
    """Sorted distinct rows: the first and last of every 256-row tile plus seeded random ones."""
    rows = {0, m - 1}
    for t in range(0, m, 256):
        rows.update({t, min(m - 1, t + 255)})
    g = seeded(seed)
    while len(rows) < min(m, count):
        rows.add(int(torch.randint(0, m, (1,), generator=g)))
    return torch.tensor(sorted(rows))


def oracle(x, rows, w_ref, b=None):
    y = x[rows].double().cpu() @ w_ref.double().t()
    return y if b is None else y + b.double().cpu()


def check_close(y, ref, what):
    y = y.double().cpu()
    err = (y - ref).abs().max().item()
    assert err <= MAX_REL * ref.abs().max().item(), f"{what}: max abs err {err} vs max {ref.abs().max().item()}"
    rel = ((y - ref).norm() / ref.norm()).item()
    assert rel <= L2_REL, f"{what}: relative L2 {rel}"
    return rel


def lin(x, e, b=None):
    return nf4_linear(x, e.parts["packed"], e.parts["absmax"], 64, codecs.NF4_CODE, e.shape, b)


def test_single_block_linear1_with_gelu_into_linear2_input(dev):
    n1 = 3 * D + MLP
    e1, w1 = weight(n1, D, 100, dev)
    x1, b1 = act(M, D, 2, dev), bias(n1, 1, dev)
    cat = torch.full((M, D + MLP), float("nan"), dtype=torch.bfloat16, device=dev)
    ((qkv, g),) = nf4_linear_gelu([(x1, e1.parts["packed"], e1.parts["absmax"], 64, codecs.NF4_CODE, e1.shape, b1,
                                    MLP, cat[:, D:])])
    assert qkv.shape == (M, 3 * D) and g.data_ptr() == cat[:, D:].data_ptr()
    rows = sample_rows(M)
    ref = oracle(x1, rows, w1, b1)
    check_close(qkv[rows], ref[:, :3 * D], "linear1 qkv columns")
    # GELU columns against the oracle GELU of the exact product (within the same bound) ...
    ref_g = S.gelu(ref[:, 3 * D:].float()).double()
    check_close(cat[rows, D:], ref_g, "linear1 GELU columns")
    # ... and bit for bit against the plain linear followed by the GELU kernel
    full = lin(x1, e1, b1)
    assert torch.equal(full[:, :3 * D], qkv)
    assert torch.equal(Kernels().gelu(full[:, 3 * D:]), cat[:, D:])
    assert torch.isnan(cat[:, :D].float()).all()  # the attention columns are left to the attention kernel


def test_single_block_linear2(dev):
    e2, w2 = weight(D, D + MLP, 200, dev)
    x2, b2 = act(M, D + MLP, 3, dev), bias(D, 2, dev)
    y = lin(x2, e2, b2)
    rows = sample_rows(M, seed=1)
    check_close(y[rows], oracle(x2, rows, w2, b2), "linear2")
    # a strided input (the [attention | GELU(mlp)] buffer as a view with a wider row) gives the same bits
    wide = torch.zeros(M, D + MLP + 64, dtype=torch.bfloat16, device=dev)
    wide[:, :D + MLP] = x2
    assert torch.equal(lin(wide[:, :D + MLP], e2, b2), y)


def test_double_block_pairs_in_one_batched_launch(dev):
    # img/txt qkv (9216 x 3072) and mlp.2 (3072 x 12288) pairs at 4096 / 512 tokens, batched as the double
    # block runs them; each must equal its own launch bit for bit and match the oracle.
    cases = [((3 * D, D), 300), ((D, MLP), 400)]
    for (n, k), seed in cases:
        ei, wi = weight(n, k, seed, dev)
        et, wt = weight(n, k, seed + 1, dev)
        xi, xt = act(4096, k, seed + 2, dev), act(512, k, seed + 3, dev)
        bi, bt = bias(n, seed + 4, dev), bias(n, seed + 5, dev)
        yi, yt = nf4_linear_batched([(xi, ei.parts["packed"], ei.parts["absmax"], 64, codecs.NF4_CODE, ei.shape, bi),
                                     (xt, et.parts["packed"], et.parts["absmax"], 64, codecs.NF4_CODE, et.shape, bt)])
        assert torch.equal(yi, lin(xi, ei, bi)) and torch.equal(yt, lin(xt, et, bt))
        ri, rt = sample_rows(4096, seed=seed), sample_rows(512, count=128, seed=seed)
        check_close(yi[ri], oracle(xi, ri, wi, bi), f"img {n}x{k}")
        check_close(yt[rt], oracle(xt, rt, wt, bt), f"txt {n}x{k}")


def test_double_block_mlp0_gelu_pair(dev):
    # img_mlp.0 / txt_mlp.0 (12288 x 3072) with the whole output through the GELU epilogue, batched.
    ei, wi = weight(MLP, D, 500, dev)
    et, wt = weight(MLP, D, 501, dev)
    xi, xt = act(4096, D, 502, dev), act(512, D, 503, dev)
    bi, bt = bias(MLP, 504, dev), bias(MLP, 505, dev)
    (ni, gi), (nt, gt) = nf4_linear_gelu([(xi, ei.parts["packed"], ei.parts["absmax"], 64, codecs.NF4_CODE, ei.shape,
                                           bi, MLP, None),
                                          (xt, et.parts["packed"], et.parts["absmax"], 64, codecs.NF4_CODE, et.shape,
                                           bt, MLP, None)])
    assert ni is None and nt is None
    k = Kernels()
    assert torch.equal(gi, k.gelu(lin(xi, ei, bi))) and torch.equal(gt, k.gelu(lin(xt, et, bt)))
    ri = sample_rows(4096, seed=7)
    check_close(gi[ri], S.gelu(oracle(xi, ri, wi, bi).float()).double(), "img mlp.0 GELU")


def test_1536_token_linear(dev):
    # 512^2 token count (1024 image + 512 text), weight 12288 x 3072, no bias: all rows checked.
    e, w = weight(4 * D, D, 0, dev)
    x = act(1536, D, 1, dev)
    y = lin(x, e)
    rows = torch.arange(1536)
    check_close(y, oracle(x, rows, w), "1536-token linear")
    # the decode of the same parts is the reference decode bit for bit
    wd = codecs.decode("nf4", e.parts, e.meta, e.shape, torch.bfloat16).cpu()
    assert torch.equal(wd.float(), w)
    assert np.isfinite(y.float().cpu().numpy()).all()


def assert_split_tail(y, alone, tail_rows, tail_cols, what):
    """y from a launch whose last round ran split (the K ranges of the tail tiles summed afterwards), against
    the same rows launched alone without a split: bit-equal outside the tail tiles, and inside them equal up
    to the rounding of the fp32 partial sums (a different summation order over K)."""
    outside = torch.ones_like(y, dtype=torch.bool)
    outside[tail_rows, tail_cols] = False
    assert torch.equal(y[outside], alone[outside]), f"{what}: whole tiles differ from the unsplit launch"
    a, b = y[tail_rows, tail_cols].double(), alone[tail_rows, tail_cols].double()
    assert ((a - b).norm() / b.norm()).item() < 1e-4, f"{what}: split tiles"
    assert (a - b).abs().max().item() <= 2.0 ** -6 * b.abs().max().item(), f"{what}: split tiles"


def test_512_batch4_linear2_split_tail(dev):
    # 4 x (1024 + 512) tokens: 24 x 12 = 288 tiles of 256 x 256, one round plus 32 tiles. On 256 CUs the
    # last 32 tiles (rows 5120-6143, columns 1024-3071 in the tile order) run as 8 K ranges of 30 blocks.
    m = 4 * 1536
    e2, w2 = weight(D, D + MLP, 600, dev)
    x2, b2 = act(m, D + MLP, 601, dev), bias(D, 602, dev)
    y = lin(x2, e2, b2)
    assert torch.equal(lin(x2, e2, b2), y)  # the partial sums are added in a fixed order
    rows = sample_rows(m, seed=3)
    check_close(y[rows], oracle(x2, rows, w2, b2), "linear2 at 512^2 batch 4")
    alone = torch.cat([lin(x2[:5120], e2, b2), lin(x2[5120:], e2, b2)])  # 240 and 48 tiles: no split
    assert_split_tail(y, alone, slice(5120, m), slice(1024, D), "linear2 at 512^2 batch 4")


def test_512_batch4_mlp2_pair_split_tail(dev):
    # The double block's mlp.2 pair at 512^2 batch 4 (4096 image, 2048 text tokens, K = 12288) in one batched
    # launch: 192 + 96 tiles, the last 32 of the text problem (its rows 1024-2047, columns 1024-3071) split.
    ei, wi = weight(D, MLP, 610, dev)
    et, wt = weight(D, MLP, 611, dev)
    xi, xt = act(4096, MLP, 612, dev), act(2048, MLP, 613, dev)
    bi, bt = bias(D, 614, dev), bias(D, 615, dev)
    yi, yt = nf4_linear_batched([(xi, ei.parts["packed"], ei.parts["absmax"], 64, codecs.NF4_CODE, ei.shape, bi),
                                 (xt, et.parts["packed"], et.parts["absmax"], 64, codecs.NF4_CODE, et.shape, bt)])
    assert torch.equal(yi, lin(xi, ei, bi))
    assert_split_tail(yt, lin(xt, et, bt), slice(1024, 2048), slice(1024, D), "text mlp.2")
    ri, rt = sample_rows(4096, seed=8), sample_rows(2048, count=128, seed=9)
    check_close(yi[ri], oracle(xi, ri, wi, bi), "img mlp.2")
    check_close(yt[rt], oracle(xt, rt, wt, bt), "txt mlp.2")
