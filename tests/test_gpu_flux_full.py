"""FLUX-dev-shaped blocks, modulations and steps on the GPU against the oracle (hidden 3072, 24 heads x 128,
mlp 12288, 512 text + 4096 image tokens at 1024^2; 1024 + 512 at 512^2).

The oracle (oracle/flux.py, pinned by goldens the reference's own functions wrote) runs on the CPU with the
reference's bf16 arithmetic: the same decoded NF4 operands, activations cast to bf16 where
selas/models/flux.py:164-200 casts them, linears with fp32 accumulation and one rounding, attention with
bf16 probabilities as torch's flash backends. Block outputs are compared on the residual update
(out - in), relative L2 <= 4e-3, the path's tolerance.
"""

from __future__ import annotations

import pytest
import torch

from oracle import flux as OF
from oracle import nf4 as onf4
from oracle import segments as S
from selas_amd import flux as F

from .conftest import seeded

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
CFG = F.FluxConfig()
OCFG = OF.FluxConfig()
L2_REL = 4e-3


def rel(a, b):
    return ((a.double().cpu() - b.double().cpu()).norm() / b.double().cpu().norm()).item()


def oracle_unit(view, dtype=BF16):
    enc = {n: (e.codec, e.shape, e.meta, {k: v.cpu() for k, v in e.parts.items()}) for n, e in view.tensors.items()}
    return OF.OracleUnit.from_encoded(enc, dtype)


@pytest.fixture(scope="module")
def flux():
    """FLUX-dev shaped, random NF4 weights, all 19 + 38 blocks and their modulation linears resident."""
    m = F.RandomFlux(CFG, "cuda", BF16, seed=0)
    yield m
    del m
    torch.cuda.empty_cache()


def rope(lt, grid):
    ids = torch.cat((torch.zeros(lt, 3), F.image_ids(grid, grid)), dim=0)
    return S.rope_tables(ids, CFG.axes_dim, CFG.theta)


def test_full_width_double_block(flux):
    lt, grid = 512, 64
    g = seeded(41)
    img = torch.randn(1, grid * grid, CFG.hidden, generator=g)
    txt = torch.randn(1, lt, CFG.hidden, generator=g)
    mod = (torch.randn(1, 12 * CFG.hidden, generator=g) * 0.3).to(BF16)
    cos, sin = rope(lt, grid)
    dev = torch.device("cuda")
    w = flux.doubles[3]
    gi, gt = F.double_block(w, img.to(dev), txt.to(dev), mod.to(dev), cos.to(dev), sin.to(dev), CFG, BF16, False)
    ri, rt = OF.double_block(oracle_unit(w), img, txt, mod, cos, sin, OCFG, BF16, False)
    ei, et = rel(gi.cpu() - img, ri - img), rel(gt.cpu() - txt, rt - txt)
    print(f"double block 1024^2: update rel L2 img {ei:.2e} txt {et:.2e}")
    assert ei <= L2_REL and et <= L2_REL


def test_full_width_single_block(flux):
    lt, grid = 512, 64
    g = seeded(42)
    x = torch.randn(1, lt + grid * grid, CFG.hidden, generator=g)
    mod = (torch.randn(1, 3 * CFG.hidden, generator=g) * 0.3).to(BF16)
    cos, sin = rope(lt, grid)
    dev = torch.device("cuda")
    w = flux.singles[5]
    gx = F.single_block(w, x.to(dev), mod.to(dev), cos.to(dev), sin.to(dev), CFG, BF16, False)
    rx = OF.single_block(oracle_unit(w), x, mod, cos, sin, OCFG, BF16, False)
    e = rel(gx.cpu() - x, rx - x)
    print(f"single block 1024^2: update rel L2 {e:.2e}")
    assert e <= L2_REL


def test_full_width_double_block_512_batch4(flux):
    # 4 images at 512^2: the image/text pairs run batched (4096 + 2048 rows), and mlp.2 (K = 12288, 288
    # tiles) runs its last 32 tiles split over K on 256 CUs.
    lt, grid, b = 512, 32, 4
    g = seeded(48)
    img = torch.randn(b, grid * grid, CFG.hidden, generator=g)
    txt = torch.randn(b, lt, CFG.hidden, generator=g)
    mod = (torch.randn(b, 12 * CFG.hidden, generator=g) * 0.3).to(BF16)
    cos, sin = rope(lt, grid)
    dev = torch.device("cuda")
    w = flux.doubles[7]
    gi, gt = F.double_block(w, img.to(dev), txt.to(dev), mod.to(dev), cos.to(dev), sin.to(dev), CFG, BF16, False)
    ri, rt = OF.double_block(oracle_unit(w), img, txt, mod, cos, sin, OCFG, BF16, False)
    ei, et = rel(gi.cpu() - img, ri - img), rel(gt.cpu() - txt, rt - txt)
    print(f"double block 512^2 batch 4: update rel L2 img {ei:.2e} txt {et:.2e}")
    assert ei <= L2_REL and et <= L2_REL


def test_full_width_single_block_512_batch4(flux):
    # 4 images at 512^2 (512 text + 1024 image tokens each, 6144 rows): linear2 (K = 15360) has 288 tiles,
    # and on 256 CUs its last 32 run split over K with their partial tiles summed by a second kernel.
    lt, grid, b = 512, 32, 4
    g = seeded(47)
    x = torch.randn(b, lt + grid * grid, CFG.hidden, generator=g)
    mod = (torch.randn(b, 3 * CFG.hidden, generator=g) * 0.3).to(BF16)
    cos, sin = rope(lt, grid)
    dev = torch.device("cuda")
    w = flux.singles[9]
    gx = F.single_block(w, x.to(dev), mod.to(dev), cos.to(dev), sin.to(dev), CFG, BF16, False)
    rx = OF.single_block(oracle_unit(w), x, mod, cos, sin, OCFG, BF16, False)
    e = rel(gx.cpu() - x, rx - x)
    print(f"single block 512^2 batch 4: update rel L2 {e:.2e}")
    assert e <= L2_REL


def test_grouped_modulations_all_76_weights(flux):
    # One grouped launch over the 76 modulation linears (19 x img/txt 3072 -> 18432, 38 x 3072 -> 9216) at
    # M = 28 steps; per weight, 96 sampled output features (all 28 rows) against the oracle's decode of those
    # rows, and a few weights against their own single launch bit for bit.
    dev = torch.device("cuda")
    sv = torch.nn.functional.silu(torch.randn(28, 1, CFG.hidden, generator=seeded(43))).to(BF16)
    mods = flux.modulations(sv.to(dev))
    assert len(mods) == 57
    pre = flux.mod_prefixes()
    assert len(pre) == 76
    outs = []
    for i, m in enumerate(mods):
        if i < 19:
            outs += [m[..., :6 * CFG.hidden], m[..., 6 * CFG.hidden:]]
        else:
            outs.append(m)
    x = sv.reshape(28, CFG.hidden).double()
    g = seeded(44)
    worst = 0.0
    for (u, p), y in zip(pre, outs):
        e = u.tensors[p + ".weight"]
        n, k = e.shape
        rows = torch.randperm(n, generator=g)[:96].sort().values
        packed = e.parts["packed"].view(n, k // 2)[rows.to(dev)].cpu().numpy().reshape(-1)
        absmax = e.parts["absmax"].view(n, k // 64)[rows.to(dev)].cpu().numpy().reshape(-1)
        w = torch.from_numpy(onf4.bf16_to_f32(onf4.c_decode(packed, absmax, 64, out=onf4.BF16))).view(-1, k)
        b = u.tensors[p + ".bias"].parts["data"][rows.to(dev)].double().cpu()
        ref = x @ w.double().t() + b
        got = y.reshape(28, n)[:, rows.to(dev)].double().cpu()
        assert (got - ref).abs().max() <= 1e-2 * ref.abs().max()
        r = ((got - ref).norm() / ref.norm()).item()
        worst = max(worst, r)
        assert r <= L2_REL, (p, r)
    print(f"76 modulation linears: worst rel L2 {worst:.2e}")
    for j in (0, 1, 37, 75):
        u, p = pre[j]
        assert torch.equal(u.linear(sv.to(dev), p).reshape(28, -1), outs[j].reshape(28, -1))


def test_57_block_step_at_1024(flux):
    # The FLUX-dev-shaped step through the runner: prepare (svec, grouped modulations, final_mod, txt_in,
    # RoPE from ids), one step, the Euler update; the velocity must be finite and shaped [1, 4096, 64].
    dev = torch.device("cuda")
    run = F.FluxRunner(flux)
    g = seeded(45)
    sig = F.get_schedule(28, 4096)
    pooled = torch.randn(1, CFG.vec_dim, generator=g)
    txt = torch.randn(1, 512, CFG.context_dim, generator=g) * 0.5
    lat = torch.randn(1, 4096, 64, generator=g).to(dev)
    cond = run.prepare(sig, 3.5, pooled, txt, F.image_ids(64, 64), F.text_ids(512))
    assert set(cond.mods) == set(run.main) and cond.mods["double.0"].shape == (28, 1, 12 * CFG.hidden)
    assert cond.final_mod.shape == (28, 1, 2 * CFG.hidden) and cond.txt.shape == (1, 512, CFG.hidden)
    v, info = run.step(0, lat, cond)
    assert v.shape == (1, 4096, 64) and v.dtype == torch.float32 and info.decision == "full"
    assert torch.isfinite(v).all() and v.abs().max() > 0
    x1 = F.euler_update(lat, sig, 0, v)
    assert torch.isfinite(x1).all()


def test_batch4_512_step_equals_images_one_by_one(flux):
    # B4 at 512^2 (1024 image + 512 text tokens per image): every kernel works per token or per
    # (image, head), so each image's velocity in the batch equals its velocity alone up to the order of
    # fp32 sums: the raw global linears img_in / txt_in / final_layer run on the library GEMM, whose
    # algorithm depends on M, and at 4 x 1536 tokens the NF4 linears with K = 12288 and 15360 run their
    # last round of tiles split over K (~6e-5 relative in the split tiles, which hold tokens of images 2
    # and 3). Through 57 random-weight blocks that grows to 7.2e-3 for images 2 and 3 (5e-5 and 2e-5 for
    # images 0 and 1; all four below 6e-5 without the split); an image reading another image's tokens or
    # modulations would differ by O(1).
    dev = torch.device("cuda")
    run = F.FluxRunner(flux)
    g = seeded(46)
    b, lt, grid = 4, 512, 32
    sig = F.get_schedule(28, grid * grid)
    pooled = torch.randn(b, CFG.vec_dim, generator=g)
    txt = torch.randn(b, lt, CFG.context_dim, generator=g) * 0.5
    lat = torch.randn(b, grid * grid, 64, generator=g).to(dev)
    cond = run.prepare(sig, 3.5, pooled, txt, F.image_ids(grid, grid), F.text_ids(lt))
    s = 3
    v, _ = run.step(s, lat, cond)
    assert v.shape == (b, grid * grid, 64) and torch.isfinite(v).all()
    for i in range(b):
        ci = run.prepare(sig, 3.5, pooled[i:i + 1], txt[i:i + 1], F.image_ids(grid, grid), F.text_ids(lt))
        assert torch.equal(ci.mods["single.7"][:, 0], cond.mods["single.7"][:, i])  # per-image modulations
        vi, _ = run.step(s, lat[i:i + 1], ci)
        assert rel(v[i:i + 1], vi) < 3e-2


def test_runner_against_the_oracle_runner():
    # A two-double, two-single-block model at hidden 256: prepare and two steps with Euler updates against
    # the oracle's prepare / step / euler (the reference's FluxRunner, pinned by its own golden) in bf16.
    cfg = F.FluxConfig(hidden=256, heads=2, mlp_hidden=1024, depth_double=2, depth_single=2, in_channels=64,
                       context_dim=128, vec_dim=64, axes_dim=(16, 56, 56))
    ocfg = OF.FluxConfig(hidden=256, heads=2, mlp_hidden=1024, depth_double=2, depth_single=2, in_channels=64,
                         context_dim=128, vec_dim=64, axes_dim=(16, 56, 56))
    model = F.RandomFlux(cfg, "cuda", BF16, seed=7)
    run = F.FluxRunner(model)
    dev = torch.device("cuda")
    g = seeded(47)
    b, lt, grid = 2, 64, 8
    sig = F.get_schedule(4, grid * grid)
    pooled = torch.randn(b, cfg.vec_dim, generator=g)
    txt = torch.randn(b, lt, cfg.context_dim, generator=g)
    lat = torch.randn(b, grid * grid, 64, generator=g)
    cond = run.prepare(sig, 4.0, pooled, txt, F.image_ids(grid, grid), F.text_ids(lt))
    og = oracle_unit(model.globals)
    mods = [oracle_unit(u) for u in model.mods]
    svecs = [OF.svec(og, ocfg, sig, 4.0, pooled[i:i + 1], BF16) for i in range(b)]
    for i in range(b):
        assert rel(run.svec(sig, 4.0, pooled[i:i + 1]), svecs[i]) < L2_REL
    per = OF.modulations(mods, svecs, 2)
    omods = [torch.cat([p[j] for p in per], dim=1) for j in range(4)]
    for j, n in enumerate(run.main):
        assert rel(cond.mods[n], omods[j]) < L2_REL, n
    ocond = OF.prepare(og, ocfg, sig, 4.0, pooled, txt, F.image_ids(grid, grid), torch.zeros(lt, 3), omods, BF16)
    assert rel(cond.final_mod, ocond.final_mod) < L2_REL and rel(cond.txt, ocond.txt) < L2_REL
    doubles = [oracle_unit(u) for u in model.doubles]
    singles = [oracle_unit(u) for u in model.singles]
    x, ox = lat.to(dev), lat
    for s in range(2):
        v, _ = run.step(s, x, cond)
        ov = OF.step(og, doubles, singles, ocfg, s, ox, ocond, BF16)
        e = rel(v, ov)
        print(f"runner step {s}: velocity rel L2 {e:.2e}")
        assert e <= L2_REL
        x, ox = F.euler_update(x, sig, s, v), OF.euler(ox, sig, s, ov)
    assert rel(x, ox) <= L2_REL
    with pytest.raises(FloatingPointError):
        F.euler_update(x, sig, 2, v * float("inf"))


def test_full_width_runner_against_the_oracle_runner():
    # FLUX-dev width (hidden 3072, 24 heads x 128, mlp 12288, context 4096, vec 768) with two double and
    # two single blocks, batch 1 at 1024^2 (512 text + 4096 image tokens): the runner's prepare and two
    # steps with Euler updates against the oracle's prepare / step / euler. This runs at real width what
    # the per-block tests leave out: img_in, the chained gated_add_mod between blocks of one kind, the
    # double -> single hand-off (cat(txt, img)), final_layer and the sampler update.
    # Two oracles on the same decoded NF4 operands: the reference's bf16 arithmetic, and exact fp32 math.
    # After four blocks the bf16 roundings (each GEMM output, each attention probability) add up to a few
    # 1e-3 of the velocity, whichever order the sums take, so the bound is stated against the exact math:
    # the GPU's distance from it is at most 1.25x the reference bf16 path's own distance, and the GPU
    # stays within 1e-2 of the reference bf16 path.
    model = F.RandomFlux(CFG, "cuda", BF16, seed=11, n_double=2, n_single=2)
    run = F.FluxRunner(model)
    dev = torch.device("cuda")
    g = seeded(48)
    lt, grid = 512, 64
    sig = F.get_schedule(28, grid * grid)
    pooled = torch.randn(1, CFG.vec_dim, generator=g)
    txt = torch.randn(1, lt, CFG.context_dim, generator=g) * 0.5
    lat = torch.randn(1, grid * grid, 64, generator=g)
    cond = run.prepare(sig, 3.5, pooled, txt, F.image_ids(grid, grid), F.text_ids(lt))
    ocfg = OF.FluxConfig(depth_double=2, depth_single=2)
    og = oracle_unit(model.globals)
    mods = [oracle_unit(u) for u in model.mods]
    doubles = [oracle_unit(u) for u in model.doubles]
    singles = [oracle_unit(u) for u in model.singles]

    def f32(u):
        return OF.OracleUnit(u.t, torch.float32)  # the same operand values, fp32 activations

    def oracle_cond(dt, gu, mu):
        sv = OF.svec(gu, ocfg, sig, 3.5, pooled, dt)
        omods = OF.modulations(mu, [sv], 2)[0]
        return sv, OF.prepare(gu, ocfg, sig, 3.5, pooled, txt, F.image_ids(grid, grid), torch.zeros(lt, 3), omods, dt)

    sv, ocond = oracle_cond(BF16, og, mods)
    _, ocond32 = oracle_cond(torch.float32, f32(og), [f32(u) for u in mods])
    assert rel(run.svec(sig, 3.5, pooled), sv) < L2_REL
    for j, n in enumerate(run.main):
        assert rel(cond.mods[n], ocond.mods[j]) < L2_REL, n
    assert rel(cond.final_mod, ocond.final_mod) < L2_REL and rel(cond.txt, ocond.txt) < L2_REL
    x, ox = lat.to(dev), lat
    for s in (0, 1):
        print(f"full-width runner step {s}: GPU step", flush=True)
        v, _ = run.step(s, x, cond)
        assert v.shape == (1, grid * grid, 64)
        print(f"full-width runner step {s}: oracle steps on the CPU (bf16, fp32)", flush=True)
        ov = OF.step(og, doubles, singles, ocfg, s, ox, ocond, BF16)
        ov32 = OF.step(f32(og), [f32(u) for u in doubles], [f32(u) for u in singles], ocfg, s, ox, ocond32,
                       torch.float32)
        gpu_exact, ref_exact, gpu_ref = rel(v, ov32), rel(ov, ov32), rel(v, ov)
        print(f"full-width runner step {s}: velocity rel L2 GPU-exact {gpu_exact:.2e}, reference bf16-exact "
              f"{ref_exact:.2e}, GPU-reference bf16 {gpu_ref:.2e}", flush=True)
        assert gpu_exact <= 1.25 * ref_exact and gpu_ref <= 1e-2
        x, ox = F.euler_update(x, sig, s, v), OF.euler(ox, sig, s, ov)
        e = rel(x - lat.to(dev), ox - lat)  # the update itself, not the latents it is added to
        print(f"full-width runner step {s}: latent update rel L2 {e:.2e}", flush=True)
        assert e <= 1e-2
    del model
    torch.cuda.empty_cache()


def test_runner_micro_batches_block_by_block():
    # FluxRunner(micro_batch=m) runs each block over chunks of at most m images (flux.py:492-524). Every
    # kernel works per token or per (image, head), and these shapes launch no split tiles, so the
    # velocity has the bits of the unchunked step for chunks of 2 (3 images: 2 + 1) and of 1.
    cfg = F.FluxConfig(hidden=256, heads=2, mlp_hidden=1024, depth_double=2, depth_single=3, in_channels=64,
                       context_dim=128, vec_dim=64, axes_dim=(16, 56, 56))
    model = F.RandomFlux(cfg, "cuda", BF16, seed=9)
    g = seeded(49)
    b, lt, grid = 3, 64, 8
    sig = F.get_schedule(4, grid * grid)
    pooled = torch.randn(b, cfg.vec_dim, generator=g)
    txt = torch.randn(b, lt, cfg.context_dim, generator=g)
    lat = torch.randn(b, grid * grid, 64, generator=g).cuda()
    whole = F.FluxRunner(model)
    cond = whole.prepare(sig, 4.0, pooled, txt, F.image_ids(grid, grid), F.text_ids(lt))
    v, _ = whole.step(1, lat, cond)
    for mb in (2, 1):
        vm, _ = F.FluxRunner(model, micro_batch=mb).step(1, lat, cond)
        assert torch.equal(vm, v), mb
    with pytest.raises(ValueError):
        F.FluxRunner(model, micro_batch=0)
