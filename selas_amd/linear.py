"""The quantized-linear forward, with the reference's ``UnitView`` interface.

The reference decodes an NF4 weight to a bf16 temporary and calls ``F.linear``
(selas/store.py:289-293, codecs.py:269-280). ``nf4_linear`` computes the same
``x @ W.T + b`` with the decode fused into the GEMM operand load, so the
decoded weight never reaches memory. Shapes outside the fused kernels
(blocksize other than 64, K not a multiple of 64, dtypes other than bf16,
misaligned rows) keep the reference's convention: the weight is decoded (on the
GPU, by the bit-exact decode kernel) and a library GEMM runs.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _lib
from .codecs import EncodedTensor, decode, int8_row_dequant, nf4_dequant


def _rows(x: torch.Tensor) -> torch.Tensor:
    """x as a 2-D [rows, K] view with unit column stride (copied only if no such view exists)."""
    k = x.shape[-1]
    if x.dim() == 2 and x.stride(-1) == 1:
        return x
    try:
        v = x.view(-1, k)
        if v.stride(-1) == 1:
            return v
    except RuntimeError:
        pass
    return x.reshape(-1, k).contiguous()


def _check_nf4_parts(packed: torch.Tensor, absmax: torch.Tensor, numel: int, blocksize: int) -> None:
    """The kernels read N*K/2 code bytes and N*K/blocksize fp32 scales from the parts' base pointers."""
    if packed.dtype != torch.uint8 or not packed.is_contiguous() or packed.numel() * 2 != numel:
        raise ValueError(f"packed NF4 data must be contiguous uint8 with {numel // 2} bytes, got {packed.dtype} "
                         f"{tuple(packed.shape)}")
    if blocksize <= 0 or numel % blocksize:
        raise ValueError(f"nf4 needs numel divisible by blocksize ({numel} % {blocksize})")
    if absmax.dtype != torch.float32 or not absmax.is_contiguous() or absmax.numel() != numel // blocksize:
        raise ValueError(f"NF4 absmax must be contiguous float32 with {numel // blocksize} values, got "
                         f"{absmax.dtype} {tuple(absmax.shape)}")


def _check_int8_parts(q: torch.Tensor, scale: torch.Tensor, n: int, k: int) -> None:
    if q.dtype != torch.int8 or not q.is_contiguous() or q.numel() != n * k:
        raise ValueError(f"int8_row data must be contiguous int8 with {n * k} values, got {q.dtype} {tuple(q.shape)}")
    if scale.dtype != torch.float32 or not scale.is_contiguous() or scale.numel() != n:
        raise ValueError(f"int8_row scale must be contiguous float32 with {n} values, got {scale.dtype} "
                         f"{tuple(scale.shape)}")


def _check_bias(bias: torch.Tensor | None, n: int) -> None:
    if bias is not None and bias.numel() != n:
        raise ValueError(f"bias has {bias.numel()} values, the weight has {n} rows")


def nf4_linear(x: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor, blocksize: int, code, shape,
               bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, decode(W), bias)`` for an NF4 weight ``W`` of ``shape`` [N, K]."""
    n, k = int(shape[0]), int(shape[1])
    if len(shape) != 2:
        raise ValueError(f"linear weight must be 2-D, got {tuple(shape)}")
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects {k}")
    dev = _lib.require_gpu(x, packed, absmax, bias)
    _check_nf4_parts(packed, absmax, n * k, int(blocksize))
    x2 = _rows(x)
    m = x2.shape[0]
    y = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
    if bias is not None and (bias.dtype != x.dtype or not bias.is_contiguous()):
        bias = bias.to(x.dtype).contiguous()
    _check_bias(bias, n)
    try:
        if x.dtype not in _lib.DTYPE_CODES:
            raise _lib.Unsupported(f"dtype {x.dtype}")
        ws, ws_bytes = _lib.workspace(_lib.CODEC_NF4, ((m, k, n),), dev) if m > 32 else (None, 0)
        with torch.cuda.device(dev):
            _lib.call("selas_nf4_linear", x2.data_ptr(), m, k, x2.stride(0), packed.data_ptr(), absmax.data_ptr(),
                      int(blocksize), _lib.code_array(code), n, _lib.ptr(bias), y.data_ptr(), n,
                      _lib.dtype_code(x.dtype), _lib.ptr(ws), ws_bytes, _lib.stream(dev))
        return y
    except _lib.Unsupported:
        w = nf4_dequant(packed, absmax, blocksize, code, (n, k), x.dtype)
        return F.linear(x, w, bias)


def int8_row_linear(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor, shape,
                    bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, decode(W), bias)`` for an int8_row weight ``W`` of ``shape`` [N, K] (q int8 [N, K],
    one fp32 scale per row). Outside the fused kernels the weight is decoded and a library GEMM runs."""
    if len(shape) != 2:
        raise ValueError(f"linear weight must be 2-D, got {tuple(shape)}")
    n, k = int(shape[0]), int(shape[1])
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects {k}")
    dev = _lib.require_gpu(x, q, scale, bias)
    _check_int8_parts(q, scale, n, k)
    x2 = _rows(x)
    m = x2.shape[0]
    y = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
    if bias is not None and (bias.dtype != x.dtype or not bias.is_contiguous()):
        bias = bias.to(x.dtype).contiguous()
    _check_bias(bias, n)
    try:
        if x.dtype not in _lib.DTYPE_CODES:
            raise _lib.Unsupported(f"dtype {x.dtype}")
        ws, ws_bytes = _lib.workspace(_lib.CODEC_INT8_ROW, ((m, k, n),), dev) if m > 32 else (None, 0)
        with torch.cuda.device(dev):
            _lib.call("selas_int8_row_linear", x2.data_ptr(), m, k, x2.stride(0), q.data_ptr(), scale.data_ptr(), n,
                      _lib.ptr(bias), y.data_ptr(), n, _lib.dtype_code(x.dtype), _lib.ptr(ws), ws_bytes,
                      _lib.stream(dev))
        return y
    except _lib.Unsupported:
        return F.linear(x, int8_row_dequant(q, scale, x.dtype).view(n, k), bias)


# Problems of the batched launches, per codec: (x, a, b, blocksize, code, shape, bias) with (a, b) =
# (packed, absmax) for NF4 and (q, scale) for int8_row (blocksize and code then unused).
def _single(codec: str, p) -> torch.Tensor:
    x, a, b, bs, code, shape, bias = p
    if codec == "nf4":
        return nf4_linear(x, a, b, bs, code, shape, bias)
    return int8_row_linear(x, a, b, shape, bias)


def _launch_batched(codec: str, arr, count: int, code, dev) -> None:
    """One tiled launch over ``arr[:count]``, with the split-tail scratch (if its plan has one) allocated here."""
    shapes = tuple((arr[i].M, arr[i].K, arr[i].N) for i in range(count) if arr[i].M > 0)
    cc = _lib.CODEC_NF4 if codec == "nf4" else _lib.CODEC_INT8_ROW
    ws, ws_bytes = _lib.workspace(cc, shapes, dev) if shapes else (None, 0)
    with torch.cuda.device(dev):
        if codec == "nf4":
            _lib.call("selas_nf4_linear_batched", ctypes.addressof(arr), count, 64, _lib.code_array(code), _lib.BF16,
                      _lib.ptr(ws), ws_bytes, _lib.stream(dev))
        else:
            _lib.call("selas_int8_row_linear_batched", ctypes.addressof(arr), count, _lib.BF16, _lib.ptr(ws), ws_bytes,
                      _lib.stream(dev))


def _batch_eligible(codec: str, problems):
    """The common codebook of NF4 problems (None for int8_row); False when the batched launch cannot take them."""
    if any(p[0].dtype != torch.bfloat16 for p in problems):
        return False
    if codec != "nf4":
        return None
    codes = {tuple(float(c) for c in p[4]) for p in problems}
    if len(codes) != 1 or any(int(p[3]) != 64 for p in problems):
        return False
    return next(iter(codes))


GROUPED_K = (1024, 2048, 3072)  # the grouped kernel keeps x in registers: K = 8 waves x 2, 4 or 6 blocks of 64
GROUPED_MAX_M = 32
GROUPED_MAX_WEIGHTS = 1023


def nf4_linear_batched(problems) -> list[torch.Tensor]:
    """``[nf4_linear(*p) for p in problems]`` with the tiled GEMMs in one launch.

    ``problems``: (x, packed, absmax, blocksize, code, shape, bias) tuples, as for
    ``nf4_linear``, with independent inputs (e.g. the image and text streams of a double
    block, selas/models/flux.py:300-324). The tiles of all problems share the GPU, so a
    small problem runs in the CUs a large one leaves idle. Each result has the bits of
    its own ``nf4_linear`` call, except in tiles that the batch's launch splits over K
    (long K with a last round of few tiles, decided from all the problems' shapes),
    whose fp32 partial sums are added in another order; when any problem is outside the
    tiled GEMM (rows <= 32, unsupported shapes) they run one by one.
    """
    return _batched("nf4", list(problems))


def int8_row_linear_batched(problems) -> list[torch.Tensor]:
    """``[int8_row_linear(*p) for p in problems]`` with the tiled GEMMs in one launch; ``problems`` are
    (x, q, scale, shape, bias) tuples. As ``nf4_linear_batched`` otherwise."""
    return _batched("int8_row", [(x, q, s, None, None, shape, b) for x, q, s, shape, b in problems])


def _batched(codec: str, problems):
    if len(problems) <= 1:
        return [_single(codec, p) for p in problems]
    outs = []
    for i in range(0, len(problems), _lib.MAX_BATCHED_LINEARS):
        outs += _batched_chunk(codec, problems[i:i + _lib.MAX_BATCHED_LINEARS])
    return outs


def _check_parts(codec: str, a: torch.Tensor, b: torch.Tensor, n: int, k: int, blocksize) -> None:
    if codec == "nf4":
        _check_nf4_parts(a, b, n * k, int(blocksize))
    else:
        _check_int8_parts(a, b, n, k)


def _batched_chunk(codec: str, problems):
    code = _batch_eligible(codec, problems)
    if code is False:
        return [_single(codec, p) for p in problems]
    dev = _lib.require_gpu(*(p[0] for p in problems), *(p[1] for p in problems))
    arr = (_lib.GemmProblem * len(problems))()
    outs, keep = [], []
    for i, (x, packed, absmax, bs, _, shape, bias) in enumerate(problems):
        n, k = int(shape[0]), int(shape[1])
        if len(shape) != 2 or x.shape[-1] != k:
            raise ValueError(f"x has {x.shape[-1]} features, weight {tuple(shape)} expects {k}")
        _check_parts(codec, packed, absmax, n, k, bs)
        x2 = _rows(x)
        if bias is not None and (bias.dtype != x.dtype or not bias.is_contiguous()):
            bias = bias.to(x.dtype).contiguous()
        _check_bias(bias, n)
        y = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
        keep += [x2, bias]
        outs.append(y)
        arr[i] = _lib.GemmProblem(x2.data_ptr(), x2.shape[0], k, x2.stride(0), packed.data_ptr(), absmax.data_ptr(), n,
                                  _lib.ptr(bias), y.data_ptr(), n)
    try:
        _launch_batched(codec, arr, len(problems), code, dev)
    except _lib.Unsupported:
        return [_single(codec, p) for p in problems]
    del keep  # the launch is queued on the stream that later reuses this memory
    return outs


def nf4_linear_gelu(problems) -> list[torch.Tensor | None]:
    """Tiled NF4 linears whose last output columns go through GELU, up to 4 per launch.

    ``problems``: (x, packed, absmax, blocksize, code, shape, bias, gelu_cols, gelu_out) tuples. For each, the
    first N - gelu_cols columns of ``x @ W.T + b`` are returned as a new tensor (None when gelu_cols == N), and
    ``gelu_out`` ([..., gelu_cols], unit column stride, equally spaced rows; allocated when None) receives
    ``gelu_tanh`` of the other columns, applied to their bf16 values: the bits of ``nf4_linear`` followed by
    the GELU segment (flux.py:194-200), without the round trip through memory. When the fused epilogue does not
    take a problem (rows <= 32, N - gelu_cols not a multiple of 256, shapes outside the tiled GEMM), that
    composition runs instead.
    """
    return _gelu("nf4", list(problems))


def int8_row_linear_gelu(problems) -> list:
    """``nf4_linear_gelu`` for int8_row weights: (x, q, scale, shape, bias, gelu_cols, gelu_out) tuples."""
    return _gelu("int8_row", [(x, q, s, None, None, shape, b, gc, out) for x, q, s, shape, b, gc, out in problems])


def _gelu(codec: str, problems):
    outs = []
    for i in range(0, len(problems), _lib.MAX_BATCHED_LINEARS):
        outs += _gelu_chunk(codec, problems[i:i + _lib.MAX_BATCHED_LINEARS])
    return outs


def _gelu_composed(codec, x, a, b, blocksize, code, shape, bias, gelu_cols, gelu_out):
    from .kernels import Kernels

    n = int(shape[0])
    y = _single(codec, (x, a, b, blocksize, code, shape, bias))
    g = Kernels().gelu(y[..., n - gelu_cols:])
    if gelu_out is None:
        gelu_out = g
    else:
        gelu_out.copy_(g)
    return (y[..., :n - gelu_cols].contiguous() if gelu_cols < n else None), gelu_out


def _gelu_chunk(codec: str, problems):
    code = _batch_eligible(codec, problems)
    if code is False:
        return [_gelu_composed(codec, *p) for p in problems]
    dev = _lib.require_gpu(*(p[0] for p in problems), *(p[1] for p in problems))
    arr = (_lib.GemmProblem * len(problems))()
    outs, keep = [], []
    for i, (x, packed, absmax, bs, _, shape, bias, gelu_cols, gelu_out) in enumerate(problems):
        n, k = int(shape[0]), int(shape[1])
        gc = int(gelu_cols)
        if len(shape) != 2 or x.shape[-1] != k or not 0 < gc <= n:
            raise ValueError(f"x has {x.shape[-1]} features, weight {tuple(shape)} expects {k}; gelu_cols {gc} "
                             f"must be in (0, {n}]")
        _check_parts(codec, packed, absmax, n, k, bs)
        x2 = _rows(x)
        if bias is not None and (bias.dtype != x.dtype or not bias.is_contiguous()):
            bias = bias.to(x.dtype).contiguous()
        _check_bias(bias, n)
        y = torch.empty(*x.shape[:-1], n - gc, dtype=x.dtype, device=dev) if gc < n else None
        if gelu_out is None:
            gelu_out = torch.empty(*x.shape[:-1], gc, dtype=x.dtype, device=dev)
        g2 = gelu_out if gelu_out.dim() == 2 else gelu_out.reshape(-1, gc) if gelu_out.is_contiguous() else None
        if g2 is None:
            lead = gelu_out.shape[:-1]
            if gelu_out.stride(-1) != 1 or any(gelu_out.stride(j) != gelu_out.stride(j + 1) * lead[j + 1]
                                               for j in range(len(lead) - 1)):
                raise ValueError(f"gelu_out rows must be equally spaced with unit column stride, strides "
                                 f"{gelu_out.stride()}")
            ldg = gelu_out.stride(-2)
        else:
            ldg = g2.stride(0)
        if gelu_out.shape[:-1] != x.shape[:-1] or gelu_out.shape[-1] != gc or gelu_out.dtype != x.dtype:
            raise ValueError(f"gelu_out must be {tuple(x.shape[:-1]) + (gc,)} {x.dtype}, got "
                             f"{tuple(gelu_out.shape)} {gelu_out.dtype}")
        keep += [x2, bias]
        outs.append((y, gelu_out))
        arr[i] = _lib.GemmProblem(x2.data_ptr(), x2.shape[0], k, x2.stride(0), packed.data_ptr(), absmax.data_ptr(), n,
                                  _lib.ptr(bias), _lib.ptr(y), n - gc, gelu_out.data_ptr(), ldg, gc)
    try:
        _launch_batched(codec, arr, len(problems), code, dev)
    except _lib.Unsupported:
        return [_gelu_composed(codec, *p[:8], o) for p, (_, o) in zip(problems, outs)]
    del keep
    return outs


class GroupedPlan:
    """A prepared grouped skinny launch: fixed NF4 (or int8_row) weights, any x with ``rows`` rows.

    ``weights``: sequence of (packed, absmax, blocksize, code, shape, bias) tuples sharing
    K; for ``codec="int8_row"`` (q, scale, None, None, shape, bias). The device descriptor
    table and the outputs are built once; ``run(x)`` is one kernel launch and returns the
    plan's own output tensors, which the next ``run`` overwrites. ``supported`` is False
    when the grouped kernel does not cover the shapes (then ``nf4_linear_grouped`` runs the
    linears one by one).
    """

    def __init__(self, weights, rows: int, device: torch.device, dtype: torch.dtype = torch.bfloat16,
                 codec: str = "nf4"):
        self.codec = codec
        self.weights = list(weights)
        self.rows = int(rows)
        self.k = int(self.weights[0][4][1]) if self.weights else 0
        self.supported = bool(self.weights) and self._eligible(dtype)
        self.outs: list[torch.Tensor] = []
        self._keep: list[torch.Tensor] = []
        self.desc = None
        if not self.supported:
            return
        rows_tbl, total_n = [], 0
        for packed, absmax, bs, _, shape, bias in self.weights:
            n = int(shape[0])
            _check_parts(codec, packed, absmax, n, self.k, 64 if bs is None else bs)
            if bias is not None and (bias.dtype != dtype or not bias.is_contiguous()):
                bias = bias.to(dtype).contiguous()
                self._keep.append(bias)
            _check_bias(bias, n)
            y = torch.empty(self.rows, n, dtype=dtype, device=device)
            self.outs.append(y)
            rows_tbl.append([packed.data_ptr(), absmax.data_ptr(), 0 if bias is None else bias.data_ptr(),
                             y.data_ptr(), n, n])
            total_n += n
        self.total_n = total_n
        self.desc = torch.tensor(rows_tbl, dtype=torch.int64).to(device)
        self.code = _lib.code_array(self.weights[0][3]) if codec == "nf4" else None

    def _eligible(self, dtype) -> bool:
        if self.codec == "nf4":
            codes = {tuple(float(c) for c in w[3]) for w in self.weights}
            if len(codes) != 1 or any(int(w[2]) != 64 for w in self.weights):
                return False
        return (dtype == torch.bfloat16 and 1 <= self.rows <= GROUPED_MAX_M and self.k in GROUPED_K
                and len(self.weights) <= GROUPED_MAX_WEIGHTS
                and all(len(w[4]) == 2 and int(w[4][1]) == self.k
                        and w[0].data_ptr() % 16 == 0 and w[1].data_ptr() % 4 == 0 for w in self.weights))

    def run(self, x: torch.Tensor) -> list[torch.Tensor]:
        """Launch for x [rows, K] (bf16, unit column stride); returns the outputs [rows, n_i]."""
        x2 = _rows(x)
        if x2.shape != (self.rows, self.k) or x2.dtype != torch.bfloat16:
            raise ValueError(f"plan expects x [{self.rows}, {self.k}] bf16, got {tuple(x2.shape)} {x2.dtype}")
        if x2.data_ptr() % 16 or x2.stride(0) % 8:
            raise ValueError("x rows must be 16-byte aligned")
        dev = _lib.require_gpu(x2, self.desc)
        with torch.cuda.device(dev):
            if self.codec == "nf4":
                _lib.call("selas_nf4_linear_grouped", x2.data_ptr(), self.rows, self.k, x2.stride(0),
                          self.desc.data_ptr(), len(self.weights), self.total_n, 64, self.code, _lib.BF16,
                          _lib.stream(dev))
            else:
                _lib.call("selas_int8_row_linear_grouped", x2.data_ptr(), self.rows, self.k, x2.stride(0),
                          self.desc.data_ptr(), len(self.weights), self.total_n, _lib.BF16, _lib.stream(dev))
        return self.outs


def nf4_linear_grouped(x: torch.Tensor, weights) -> list[torch.Tensor]:
    """``[F.linear(x, decode(W_i), b_i) for W_i, b_i in weights]`` in one launch.

    ``weights``: sequence of (packed, absmax, blocksize, code, shape, bias) tuples that
    share ``x`` [..., K] with at most 32 rows. Each result is a new tensor with the bits
    ``nf4_linear`` gives for that weight alone. This is the hoisted modulation prologue
    (selas/models/flux.py:428-445): every modulation linear of a model applied to one
    silu(vec). Shapes the grouped kernel does not cover are run one by one.
    """
    return _grouped("nf4", x, list(weights))


def int8_row_linear_grouped(x: torch.Tensor, weights) -> list[torch.Tensor]:
    """``nf4_linear_grouped`` for int8_row weights: (q, scale, shape, bias) tuples sharing ``x``."""
    return _grouped("int8_row", x, [(q, s, None, None, shape, b) for q, s, shape, b in weights])


def _grouped(codec: str, x: torch.Tensor, weights) -> list[torch.Tensor]:
    if not weights:
        return []
    dev = _lib.require_gpu(x, *(w[0] for w in weights))
    x2 = _rows(x)
    plan = GroupedPlan(weights, x2.shape[0], dev, x.dtype, codec)
    if not plan.supported or x2.data_ptr() % 16 or x2.stride(0) % 8 or x2.shape[1] != plan.k:
        return [_single(codec, (x, *w)) for w in weights]
    outs = plan.run(x2)
    # The plan's descriptor table may be freed now: the caching allocator hands its memory
    # only to later work on this same stream, which runs after the launch.
    return [y.view(*x.shape[:-1], y.shape[-1]) for y in outs]


_DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16, "uint8": torch.uint8,
           "int8": torch.int8, "int32": torch.int32, "int64": torch.int64, "float64": torch.float64}


def part_view(buf: torch.Tensor, part) -> torch.Tensor:
    """One part of a unit held in the 1-D uint8 tensor ``buf``, viewed in place with its own dtype and
    shape (selas/container.py:79-82). ``part`` has selas's PartSpec fields: offset (relative to the
    unit), nbytes, dtype (a name such as "bfloat16") and shape."""
    dt = part.dtype if isinstance(part.dtype, torch.dtype) else _DTYPES[str(part.dtype).removeprefix("torch.")]
    return buf[part.offset: part.offset + part.nbytes].view(dt).view(tuple(part.shape))


class UnitView:
    """Typed access to one unit's tensors, as selas.store.UnitView (store.py:242-293).

    Built as selas's store builds it, ``UnitView(spec, buf, dtype)``: ``spec`` has ``.tensors``
    mapping names to TensorSpec-like entries (codec, shape, meta, parts of PartSpec-like entries)
    and ``buf`` is the unit's 1-D uint8 device buffer; parts are viewed in place (part_view), never
    copied. ``UnitView(tensors, dtype)`` takes a dict of :class:`EncodedTensor` with device parts
    instead. ``get`` decodes (raw tensors in the compute dtype are returned as zero-copy views and
    cached), ``linear`` is the quantized-linear forward.
    """

    __slots__ = ("tensors", "dtype", "_views", "spec", "buf")

    def __init__(self, spec_or_tensors, buf_or_dtype, dtype: torch.dtype | None = None):
        self._views: dict[tuple, torch.Tensor] = {}
        if dtype is None:  # (tensors, dtype)
            self.spec, self.buf = None, None
            self.tensors: dict[str, EncodedTensor] = spec_or_tensors
            self.dtype = buf_or_dtype
            return
        self.spec, self.buf, self.dtype = spec_or_tensors, buf_or_dtype, dtype
        if self.buf.dtype != torch.uint8 or self.buf.dim() != 1:
            raise ValueError(f"unit buffer must be 1-D uint8, got {self.buf.dtype} {tuple(self.buf.shape)}")
        self.tensors = {name: EncodedTensor(name, ts.codec, tuple(ts.shape), dict(ts.meta),
                                            {k: part_view(self.buf, ps) for k, ps in ts.parts.items()})
                        for name, ts in self.spec.tensors.items()}

    def has(self, name: str) -> bool:
        return name in self.tensors

    def codec(self, name: str) -> str:
        return self.tensors[name].codec

    def parts(self, name: str) -> dict[str, torch.Tensor]:
        return self.tensors[name].parts

    def get(self, name: str, dtype: torch.dtype | None = None) -> torch.Tensor:
        dtype = dtype or self.dtype
        key = (name, dtype)
        hit = self._views.get(key)
        if hit is not None:
            return hit
        e = self.tensors[name]
        out = decode(e.codec, e.parts, e.meta, e.shape, dtype)
        if e.codec == "raw" and out.data_ptr() == e.parts["data"].data_ptr():
            self._views[key] = out
        return out

    def _problem(self, x: torch.Tensor, prefix: str, dtype: torch.dtype):
        """(codec, (x, a, b, blocksize, code, shape, bias)) for a fused codec, or (None, bias)."""
        e = self.tensors[prefix + ".weight"]
        bname = prefix + ".bias"
        b = self.get(bname, dtype) if bname in self.tensors else None
        if x.dtype != dtype or len(e.shape) != 2:
            return None, b
        if e.codec == "nf4":
            return "nf4", (x, e.parts["packed"], e.parts["absmax"], int(e.meta["blocksize"]), e.meta["code"], e.shape, b)
        if e.codec == "int8_row":
            return "int8_row", (x, e.parts["q"], e.parts["scale"], None, None, e.shape, b)
        return None, b

    def linear_many(self, items, dtype: torch.dtype | None = None) -> list[torch.Tensor]:
        """``[self.linear(x, prefix) for x, prefix in items]``, the tiled GEMMs of one codec in one launch."""
        dtype = dtype or self.dtype
        items = list(items)
        probs = [self._problem(x, prefix, dtype) for x, prefix in items]
        codecs = {c for c, _ in probs}
        if len(codecs) != 1 or None in codecs:
            return [self.linear(x, p, dtype) for x, p in items]
        return _batched(codecs.pop(), [p for _, p in probs])

    def linear_gelu_many(self, items, dtype: torch.dtype | None = None) -> list:
        """For (x, prefix, gelu_cols, gelu_out) items: the linear with GELU applied to its last gelu_cols
        output columns, written to gelu_out (NF4 and int8_row weights: in the GEMM epilogue, one launch per
        codec); returns (plain columns or None, gelu_out) per item."""
        dtype = dtype or self.dtype
        by_codec: dict[str, list] = {}
        results: list = []
        for i, (x, prefix, gc, out) in enumerate(items):
            codec, prob = self._problem(x, prefix, dtype)
            if codec is not None:
                by_codec.setdefault(codec, []).append((i, prob + (gc, out)))
                results.append(None)
            else:  # other weights: the linear, then the GELU segment
                from .kernels import Kernels

                y = self.linear(x, prefix, dtype)
                n = y.shape[-1]
                g = Kernels().gelu(y[..., n - gc:])
                if out is not None:
                    out.copy_(g)
                results.append((y[..., :n - gc].contiguous() if gc < n else None, out if out is not None else g))
        for codec, group in by_codec.items():
            for (i, _), r in zip(group, _gelu(codec, [p for _, p in group])):
                results[i] = r
        return results

    def linear(self, x: torch.Tensor, prefix: str, dtype: torch.dtype | None = None) -> torch.Tensor:
        dtype = dtype or self.dtype
        codec, prob = self._problem(x, prefix, dtype)
        if codec is not None:
            return _single(codec, prob)
        return F.linear(x, self.get(prefix + ".weight", dtype), prob)
