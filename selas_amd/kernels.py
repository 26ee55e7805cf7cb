"""The elementwise segments of a FLUX block as gfx950 kernels, with the reference's interface.

``Kernels`` has the seven segment methods of selas.models.flux.Kernels
(flux.py:206-212) with the same names, arguments and return values, so an
instance can be passed as ``kernels=`` to selas's FluxRunner or ``k=`` to its
block functions. Each method is one kernel launch on the current stream; the
fp32 math matches the eager segments (flux.py:164-200) up to rounding.

Where a kernel does not take a call (a width that is not a multiple of 4 or
above 4096, rows off 16-byte alignment, other dtypes or layouts), the method
warns once per segment and runs the eager segment in torch on the same GPU, as
the reference's compiled segments fall back to eager ones (flux.py:215-235).
Argument errors, HIP errors and out-of-memory are raised, never swallowed.
"""

from __future__ import annotations

import threading
import warnings

import torch
import torch.nn.functional as F

from . import _lib

SEGMENT_NAMES = ("mod_in", "gated_add", "gated_add_mod", "qkv_double", "qkv_single", "gelu", "attn_mlp")


def _bld(x: torch.Tensor, what: str) -> tuple[int, int, int, int, int]:
    """(B, L, D, batch stride, row stride) of a [B, L, D] or [L, D] tensor with unit column stride."""
    if x.dim() == 2:
        x = x.unsqueeze(0)
    if x.dim() != 3 or x.stride(-1) != 1:
        raise _lib.Unsupported(f"{what}: the kernels take [B, L, D] with contiguous D, got shape {tuple(x.shape)} "
                               f"strides {x.stride()}")
    b, l, d = x.shape
    return b, l, d, x.stride(0) if b > 1 else 0, x.stride(1) if l > 1 else d


def _vec(v: torch.Tensor, b: int, d: int, what: str) -> tuple[torch.Tensor, int]:
    """A per-batch modulation vector ([B|1, 1, D], [B|1, D] or [D]) as fp32 plus its batch stride."""
    if v.dtype != torch.float32:
        v = v.float()
    if v.shape[-1] != d or v.stride(-1) != 1:
        v = v.contiguous()
    if v.dim() == 3:
        if v.shape[1] != 1:
            raise _lib.Unsupported(f"{what}: the kernels take [B, 1, D] vectors, got {tuple(v.shape)}")
        vb, sb = v.shape[0], v.stride(0)
    elif v.dim() == 2:
        vb, sb = v.shape[0], v.stride(0)
    elif v.dim() == 1:
        vb, sb = 1, 0
    else:
        raise _lib.Unsupported(f"{what}: the kernels take [B, 1, D], [B, D] or [D] vectors, got {tuple(v.shape)}")
    if v.shape[-1] != d or vb not in (1, b):
        raise _lib.Unsupported(f"{what}: vector {tuple(v.shape)} is not one row per batch (batch {b}, width {d})")
    return v, (sb if vb > 1 else 0)


def _vec_pair(shift: torch.Tensor, scale: torch.Tensor, b: int, d: int, what: str):
    """shift and scale with one shared batch stride: where one is per batch ([B, 1, D]) and the other
    broadcast ([1, 1, D]), both are laid out per batch (a [B, D] copy of at most B*D floats)."""
    shift, msb = _vec(shift, b, d, what + " shift")
    scale, csb = _vec(scale, b, d, what + " scale")
    if msb == csb:
        return shift, scale, msb
    shift = shift.reshape(-1, d).expand(b, d).contiguous()
    scale = scale.reshape(-1, d).expand(b, d).contiguous()
    return shift, scale, d


def _f32_rows(x: torch.Tensor, what: str) -> torch.Tensor:
    if x.dtype != torch.float32:
        raise _lib.Unsupported(f"{what}: the kernels take a float32 residual stream, got {x.dtype}")
    return x


# ---------------------------------------------------------------------------- eager segments
#
# The segments as torch operations on the caller's device: the math of selas's eager
# segments (flux.py:117-147, 164-200), run when a kernel does not take a call.

_FP16_MAX = 65504.0


def _eager_ln(x):
    return F.layer_norm(x, (x.shape[-1],), eps=1e-6)


def _eager_res(y, guard):
    y = y.float()
    return y.clamp(-_FP16_MAX, _FP16_MAX) if guard else y


def _eager_mod_in(x, shift, scale, dt):
    return (_eager_ln(x) * (1 + scale) + shift).to(dt)


def _eager_gated_add(x, g, y, guard):
    return x + g * _eager_res(y, guard)


def _eager_gated_add_mod(x, g, y, shift, scale, dt, guard):
    x = _eager_gated_add(x, g, y, guard)
    return x, _eager_mod_in(x, shift, scale, dt)


def _eager_split_heads(qkv, heads):
    b, l, _ = qkv.shape
    t = qkv.view(b, l, 3, heads, -1).permute(2, 0, 3, 1, 4)  # channel = which * H * Dh + h * Dh + d
    return t[0], t[1], t[2]


def _eager_rms(x, scale):
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * scale


def _eager_rope(x, cos, sin):
    even, odd = x[..., 0::2], x[..., 1::2]  # interleaved pairs (x[2i], x[2i+1])
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1).flatten(-2)


def _eager_qkv_double(tqkv, iqkv, tqs, tks, iqs, iks, cos, sin, heads, dt):
    tq, tk, tv = _eager_split_heads(tqkv, heads)
    iq, ik, iv = _eager_split_heads(iqkv, heads)
    q = _eager_rope(torch.cat((_eager_rms(tq, tqs), _eager_rms(iq, iqs)), dim=2), cos, sin).to(dt)
    k = _eager_rope(torch.cat((_eager_rms(tk, tks), _eager_rms(ik, iks)), dim=2), cos, sin).to(dt)
    return q, k, torch.cat((tv, iv), dim=2)


def _eager_qkv_single(qkv, qs, ks, cos, sin, heads, dt):
    q, k, v = _eager_split_heads(qkv, heads)
    return (_eager_rope(_eager_rms(q, qs), cos, sin).to(dt), _eager_rope(_eager_rms(k, ks), cos, sin).to(dt),
            v.contiguous())


def _eager_gelu(h):
    return F.gelu(h, approximate="tanh")


def _eager_attn_mlp(attn, mlp):
    return torch.cat((attn, _eager_gelu(mlp)), dim=2)


EAGER_SEGMENTS = {"mod_in": _eager_mod_in, "gated_add": _eager_gated_add, "gated_add_mod": _eager_gated_add_mod,
                  "qkv_double": _eager_qkv_double, "qkv_single": _eager_qkv_single, "gelu": _eager_gelu,
                  "attn_mlp": _eager_attn_mlp}

_warned: set[str] = set()
_warned_lock = threading.Lock()


def _fallback(name: str, err: Exception, args):
    """The eager segment for a call the kernel did not take, with one warning per segment and process.
    Like the kernels it runs on the GPU only: CPU tensors are an error."""
    _lib.require_gpu(*(a for a in args if isinstance(a, torch.Tensor)))
    with _warned_lock:
        first = name not in _warned
        _warned.add(name)
    if first:
        warnings.warn(f"selas_amd kernel for {name} does not take this call ({str(err).splitlines()[0][:200]}); "
                      "running the eager segment for such calls", RuntimeWarning, stacklevel=3)
    return EAGER_SEGMENTS[name](*args)


class Kernels:
    """The segments of a block (mod_in, gated_add, gated_add_mod, qkv_double, qkv_single, gelu, attn_mlp).

    Each public method runs its kernel, or the eager segment (with a one-time warning) for calls the
    kernel does not take."""

    compiled = True  # fused kernels (the reference's Kernels(compiled=True) role)

    def mod_in(self, x, shift, scale, dt):
        """``(LN(x) * (1 + scale) + shift).to(dt)`` (flux.py:164-166)."""
        try:
            return self._mod_in(x, shift, scale, dt)
        except _lib.Unsupported as e:
            return _fallback("mod_in", e, (x, shift, scale, dt))

    def gated_add(self, x, g, y, guard: bool):
        """``x + g * float(y)`` with y clamped to the fp16 range when ``guard`` (flux.py:169-171)."""
        try:
            return self._gated(x, g, y, guard, None, None, None)[0]
        except _lib.Unsupported as e:
            return _fallback("gated_add", e, (x, g, y, guard))

    def gated_add_mod(self, x, g, y, shift, scale, dt, guard: bool):
        """``(x', mod_in(x', shift, scale, dt))`` with ``x' = gated_add(x, g, y, guard)`` (flux.py:174-176)."""
        try:
            return self._gated(x, g, y, guard, shift, scale, dt)
        except _lib.Unsupported as e:
            return _fallback("gated_add_mod", e, (x, g, y, shift, scale, dt, guard))

    def qkv_single(self, qkv, qs, ks, cos, sin, heads: int, dt):
        """(q, k, v) [B, H, L, Dh] from linear1's qkv view (flux.py:188-191)."""
        try:
            return self._qkv_single(qkv, qs, ks, cos, sin, heads, dt)
        except _lib.Unsupported as e:
            return _fallback("qkv_single", e, (qkv, qs, ks, cos, sin, heads, dt))

    def qkv_double(self, tqkv, iqkv, tqs, tks, iqs, iks, cos, sin, heads: int, dt):
        """(q, k, v) [B, H, Lt+Li, Dh], text first, per-stream QK norms (flux.py:179-185)."""
        try:
            return self._qkv_double(tqkv, iqkv, tqs, tks, iqs, iks, cos, sin, heads, dt)
        except _lib.Unsupported as e:
            return _fallback("qkv_double", e, (tqkv, iqkv, tqs, tks, iqs, iks, cos, sin, heads, dt))

    def gelu(self, h):
        """GELU with the tanh approximation (flux.py:194-195)."""
        try:
            return self._gelu(h)
        except _lib.Unsupported as e:
            return _fallback("gelu", e, (h,))

    def attn_mlp(self, attn, mlp):
        """``cat((attn, gelu(mlp)), dim=2)``: linear2's input (flux.py:198-200)."""
        try:
            return self._attn_mlp(attn, mlp)
        except _lib.Unsupported as e:
            return _fallback("attn_mlp", e, (attn, mlp))

    # ------------------------------------------------------------------ LayerNorm + adaLN
    def _mod_in(self, x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
        dev = _lib.require_gpu(x, shift, scale)
        x = _f32_rows(x, "mod_in")
        b, l, d, sb, sl = _bld(x, "mod_in")
        shift, scale, msb = _vec_pair(shift, scale, b, d, "mod_in")
        out = torch.empty(*x.shape, dtype=dt, device=dev)
        with torch.cuda.device(dev):
            _lib.call("selas_mod_in", x.data_ptr(), b, l, d, sb, sl, shift.data_ptr(), scale.data_ptr(), msb,
                      out.data_ptr(), _lib.dtype_code(dt), _lib.stream(dev))
        return out

    # ------------------------------------------------------------------ gated residual
    def _gated(self, x, g, y, guard, shift, scale, dt):
        what = "gated_add" if shift is None else "gated_add_mod"
        dev = _lib.require_gpu(x, g, y, shift, scale)
        x = _f32_rows(x, what)
        b, l, d, sb, sl = _bld(x, what)
        yb, yl, yd, ysb, ysl = _bld(y, what + " y")
        if (yb, yl, yd) != (b, l, d):
            raise _lib.Unsupported(f"{what}: the kernels take y of x's shape, got {tuple(y.shape)} for "
                                   f"{tuple(x.shape)}")
        g, gsb = _vec(g, b, d, what + " gate")
        x_out = torch.empty(*x.shape, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            if shift is None:
                _lib.call("selas_gated_add", x.data_ptr(), b, l, d, sb, sl, g.data_ptr(), gsb, y.data_ptr(),
                          _lib.dtype_code(y.dtype), ysb, ysl, int(bool(guard)), x_out.data_ptr(), _lib.stream(dev))
                return x_out, None
            shift, scale, msb = _vec_pair(shift, scale, b, d, what)
            h = torch.empty(*x.shape, dtype=dt, device=dev)
            _lib.call("selas_gated_add_mod", x.data_ptr(), b, l, d, sb, sl, g.data_ptr(), gsb, y.data_ptr(),
                      _lib.dtype_code(y.dtype), ysb, ysl, int(bool(guard)), shift.data_ptr(), scale.data_ptr(), msb,
                      x_out.data_ptr(), h.data_ptr(), _lib.dtype_code(dt), _lib.stream(dev))
        return x_out, h

    # ------------------------------------------------------------------ attention prep
    @staticmethod
    def _heads_src(qkv: torch.Tensor, heads: int, what: str):
        if qkv.dim() != 3 or qkv.stride(-1) != 1:
            raise _lib.Unsupported(f"{what}: the kernels take qkv [B, L, 3*H*Dh] with contiguous channels")
        b, l, c = qkv.shape
        if c % (3 * heads):
            raise ValueError(f"{what}: {c} channels do not split into 3 x {heads} heads")
        return b, l, c // (3 * heads), qkv.stride(0) if b > 1 else 0, qkv.stride(1) if l > 1 else c

    @staticmethod
    def _scale(s: torch.Tensor, dh: int) -> torch.Tensor:
        s = s.reshape(-1)
        if s.numel() != dh:
            raise ValueError(f"norm scale has {s.numel()} values, head_dim is {dh}")
        return s.float().contiguous()

    def _qkv_single(self, qkv, qs, ks, cos, sin, heads: int, dt):
        dev = _lib.require_gpu(qkv, qs, ks, cos, sin)
        b, l, dh, sb, sl = self._heads_src(qkv, heads, "qkv_single")
        if qkv.dtype != dt:
            raise _lib.Unsupported(f"qkv_single: the kernels take qkv in the compute dtype, got {qkv.dtype} for {dt}")
        cos, sin = cos.float().contiguous(), sin.float().contiguous()
        if cos.shape != (l, dh // 2) or sin.shape != (l, dh // 2):
            raise ValueError(f"qkv_single: rope tables {tuple(cos.shape)} do not match L={l}, head_dim={dh}")
        qs, ks = self._scale(qs, dh), self._scale(ks, dh)
        q, k, v = (torch.empty(b, heads, l, dh, dtype=dt, device=dev) for _ in range(3))
        with torch.cuda.device(dev):
            _lib.call("selas_qkv_single", qkv.data_ptr(), b, l, heads, dh, sb, sl, qs.data_ptr(), ks.data_ptr(),
                      cos.data_ptr(), sin.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.dtype_code(dt),
                      _lib.stream(dev))
        return q, k, v

    def _qkv_double(self, tqkv, iqkv, tqs, tks, iqs, iks, cos, sin, heads: int, dt):
        dev = _lib.require_gpu(tqkv, iqkv, tqs, tks, iqs, iks, cos, sin)
        tb, lt, dh, tsb, tsl = self._heads_src(tqkv, heads, "qkv_double txt")
        ib, li, dhi, isb, isl = self._heads_src(iqkv, heads, "qkv_double img")
        if tb != ib or dh != dhi:
            raise ValueError(f"qkv_double: txt {tuple(tqkv.shape)} and img {tuple(iqkv.shape)} disagree")
        if tqkv.dtype != dt or iqkv.dtype != dt:
            raise _lib.Unsupported(f"qkv_double: the kernels take qkv in the compute dtype, got "
                                   f"{tqkv.dtype}/{iqkv.dtype} for {dt}")
        cos, sin = cos.float().contiguous(), sin.float().contiguous()
        if cos.shape != (lt + li, dh // 2) or sin.shape != (lt + li, dh // 2):
            raise ValueError(f"qkv_double: rope tables {tuple(cos.shape)} do not match L={lt + li}, head_dim={dh}")
        tqs, tks, iqs, iks = (self._scale(s, dh) for s in (tqs, tks, iqs, iks))
        q, k, v = (torch.empty(tb, heads, lt + li, dh, dtype=dt, device=dev) for _ in range(3))
        with torch.cuda.device(dev):
            _lib.call("selas_qkv_double", tqkv.data_ptr(), tsb, tsl, lt, iqkv.data_ptr(), isb, isl, li, tb, heads,
                      dh, tqs.data_ptr(), tks.data_ptr(), iqs.data_ptr(), iks.data_ptr(), cos.data_ptr(),
                      sin.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.dtype_code(dt), _lib.stream(dev))
        return q, k, v

    # ------------------------------------------------------------------ MLP activation
    @staticmethod
    def _rows2(t: torch.Tensor, what: str) -> tuple[int, int, int]:
        """(rows, cols, row stride) of a tensor whose leading dims collapse onto one row stride."""
        if t.stride(-1) != 1:
            raise _lib.Unsupported(f"{what}: the kernels take a contiguous last dim")
        cols = t.shape[-1]
        rows = t.numel() // cols if cols else 0
        if t.dim() == 1:
            return 1, cols, cols
        ld = t.stride(-2) if t.shape[-2] > 1 else cols
        expect = ld
        for i in range(t.dim() - 2, 0, -1):  # outer dims must be dense over rows of stride ld
            expect *= t.shape[i]
            if t.shape[i - 1] > 1 and t.stride(i - 1) != expect:
                raise _lib.Unsupported(f"{what}: the kernels take rows that share one stride")
        return rows, cols, ld

    def _gelu(self, h: torch.Tensor) -> torch.Tensor:
        dev = _lib.require_gpu(h)
        rows, cols, ld = self._rows2(h, "gelu")
        out = torch.empty(*h.shape, dtype=h.dtype, device=dev)
        with torch.cuda.device(dev):
            _lib.call("selas_gelu", h.data_ptr(), rows, cols, ld, out.data_ptr(), _lib.dtype_code(h.dtype),
                      _lib.stream(dev))
        return out

    def _attn_mlp(self, attn: torch.Tensor, mlp: torch.Tensor) -> torch.Tensor:
        dev = _lib.require_gpu(attn, mlp)
        if attn.shape[:-1] != mlp.shape[:-1] or attn.dtype != mlp.dtype:
            raise _lib.Unsupported(f"attn_mlp: attn {tuple(attn.shape)} {attn.dtype} vs mlp {tuple(mlp.shape)} {mlp.dtype}")
        ra, da, lda = self._rows2(attn, "attn_mlp attn")
        rm, dm, ldm = self._rows2(mlp, "attn_mlp mlp")
        out = torch.empty(*attn.shape[:-1], da + dm, dtype=attn.dtype, device=dev)
        with torch.cuda.device(dev):
            _lib.call("selas_attn_mlp", attn.data_ptr(), ra, da, lda, mlp.data_ptr(), dm, ldm, out.data_ptr(),
                      _lib.dtype_code(attn.dtype), _lib.stream(dev))
        return out


FUSED = Kernels()
