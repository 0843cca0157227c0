"""Scaled fp8 boundary quantization on MI355X: the drop-in for wantrain's
model/fp8.py (same names, arguments, return shapes and errors).

One power-of-two scale per row (last dim): k = frexp(amax|x|).exponent -
ebias, q = fp8(x * 2^-k), x_hat = float(q) * 2^k, bit for bit what the
reference's torch ops give (model/fp8.py:28-63).  The work runs in the gfx950
kernels of libelyhip.so; a row is read once, scaled and converted in
registers.  Per-tensor scaling is a single row: quantize(x.reshape(1, -1)),
or per_tensor=True.

Inputs must be CUDA tensors of dtype bfloat16 or float32.
"""

from __future__ import annotations

import math

import torch

from . import _lib

# fmt -> (torch dtype, e with 2^e above the format's largest finite value);
# model/fp8.py:17-20.
FORMATS = {
    "e4m3": (torch.float8_e4m3fn, 8),
    "e5m2": (torch.float8_e5m2, 15),
}

# Candidate offsets of recover_exp, in the order they are tried
# (model/fp8.py:25).
_DELTAS = (0, -1, 1, -2, 2)


def _fmt(fmt: str) -> int:
    if fmt not in FORMATS:
        raise ValueError(f"fp8 format {fmt!r} is not one of {tuple(FORMATS)}")
    return _lib.FMT[fmt]


def _rows(x: torch.Tensor, what: str):
    _lib.require_gpu(x, what)
    if x.dim() == 0:
        raise ValueError(f"{what}: a 0-d tensor has no rows")
    x = x.detach()
    if not x.is_contiguous():
        x = x.contiguous()
    cols = x.shape[-1]
    rows = math.prod(x.shape[:-1])
    return x, rows, cols


def _k_shape(x: torch.Tensor):
    return tuple(x.shape[:-1]) + (1,)


def scale_exp(x: torch.Tensor, fmt: str = "e4m3", per_tensor: bool = False) -> torch.Tensor:
    """Per-row exponent k (int32, shaped like x with the last dim 1) such that
    x * 2^-k fits the fp8 range; 0 for an all-zero row (model/fp8.py:28-38)."""
    f = _fmt(fmt)
    if per_tensor:
        return scale_exp(x.reshape(1, -1), fmt).reshape((1,) * x.dim())
    x, rows, cols = _rows(x, "scale_exp")
    k = torch.empty(_k_shape(x), dtype=torch.int32, device=x.device)
    L = _lib.load()
    ws = _lib.workspace(x.device, L.ely_fp8_workspace_bytes(rows, cols, _lib.dtype_code(x)))
    _lib.check(
        L.ely_fp8_quantize(x.data_ptr(), _lib.dtype_code(x), rows, cols, f, None, k.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(x.device)),
        "scale_exp",
    )
    return k


def _hint(k_hint, per_tensor: bool, what: str):
    """None, an int32, or a one-element int32 tensor (read on the GPU)."""
    if k_hint is None:
        return None
    if not per_tensor:
        raise ValueError(f"{what}: k_hint applies to per-tensor scaling (per_tensor=True)")
    if isinstance(k_hint, torch.Tensor):
        if k_hint.dtype != torch.int32 or k_hint.numel() != 1:
            raise ValueError(f"{what}: a k_hint tensor holds one int32 (an exponent quantize returned), got {k_hint.dtype} x {k_hint.numel()}")
        return k_hint
    k_hint = int(k_hint)
    if not -(2**31) <= k_hint < 2**31:
        raise ValueError(f"{what}: k_hint {k_hint} is not an int32")
    return k_hint


def _per_tensor_hint(x: torch.Tensor, f: int, k_hint, q, out, what: str) -> torch.Tensor:
    """The one-pass per-tensor path (ely_fp8_quantize_hint): fills q and/or
    out, returns k (one element, on x's device).  A tensor hint is read on
    the GPU, so the call does not wait for it."""
    _lib.require_gpu(x, what)
    x = x.detach().contiguous()
    dev_hint = None
    if isinstance(k_hint, torch.Tensor):
        if k_hint.device != x.device:
            raise ValueError(f"{what}: the k_hint tensor is on {k_hint.device}, x on {x.device}")
        dev_hint, k_hint = k_hint.contiguous(), 0
    k = torch.empty(1, dtype=torch.int32, device=x.device)
    L = _lib.load()
    ws = _lib.workspace(x.device, L.ely_fp8_hint_workspace_bytes(x.numel()))
    _lib.check(
        L.ely_fp8_quantize_hint(x.data_ptr(), _lib.dtype_code(x), x.numel(), f, k_hint,
                                None if dev_hint is None else dev_hint.data_ptr(), None if q is None else q.data_ptr(),
                                k.data_ptr(), None if out is None else out.data_ptr(), None, ws.data_ptr(), ws.numel(),
                                _lib.stream_ptr(x.device)),
        what,
    )
    return k


def quantize(x: torch.Tensor, fmt: str = "e4m3", per_tensor: bool = False, k_hint: int | torch.Tensor | None = None):
    """x -> (fp8 tensor shaped like x, int32 k shaped like x with the last dim
    1).  Exact given k (model/fp8.py:45-49).

    k_hint (per-tensor only; an addition to the reference's signature): the
    exponent the caller expects, e.g. the previous step's, as an int or as
    the one-element int32 tensor an earlier call returned (read on the GPU,
    no host wait).  The results are the same whatever the hint; when it is
    right, x is read once instead of twice.  Without one, a per-tensor x of
    64 MiB or more guesses its exponent from a sample of x (every 61st
    2,048-element segment) and is read once when the guess holds."""
    f = _fmt(fmt)
    hint = _hint(k_hint, per_tensor, "quantize")
    if hint is not None:
        if x.dim() == 0:
            raise ValueError("quantize: a 0-d tensor has no rows")
        q = torch.empty(x.shape, dtype=FORMATS[fmt][0], device=x.device)
        k = _per_tensor_hint(x, f, hint, q, None, "quantize")
        return q, k.reshape((1,) * x.dim())
    if per_tensor:
        q, k = quantize(x.reshape(1, -1), fmt)
        return q.reshape(x.shape), k.reshape((1,) * x.dim())
    dt, _ = FORMATS[fmt]
    x, rows, cols = _rows(x, "quantize")
    q = torch.empty(x.shape, dtype=dt, device=x.device)
    k = torch.empty(_k_shape(x), dtype=torch.int32, device=x.device)
    L = _lib.load()
    ws = _lib.workspace(x.device, L.ely_fp8_workspace_bytes(rows, cols, _lib.dtype_code(x)))
    _lib.check(
        L.ely_fp8_quantize(x.data_ptr(), _lib.dtype_code(x), rows, cols, f, q.data_ptr(), k.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(x.device)),
        "quantize",
    )
    return q, k


def _fmt_of(q: torch.Tensor) -> str:
    for name, (dt, _) in FORMATS.items():
        if q.dtype == dt:
            return name
    raise ValueError(f"dequantize takes a float8_e4m3fn or float8_e5m2 tensor, got {q.dtype}")


def dequantize(q: torch.Tensor, k: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """q.to(dtype) * 2^k, exact (model/fp8.py:52-53).  k holds one exponent
    per row of q (shape [..., 1], or one element for a per-tensor q)."""
    fmt = _fmt_of(q)
    _lib.require_gpu(q, "dequantize")
    if dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"dequantize writes float32 or bfloat16, got {dtype}")
    q = q.contiguous()
    if q.dim() == 0:
        raise ValueError("dequantize: a 0-d tensor has no rows")
    k = k.to(device=q.device, dtype=torch.int32).contiguous()
    cols = q.shape[-1]
    rows = math.prod(q.shape[:-1])
    if k.numel() == 1 and rows != 1:
        # per-tensor exponent: one row of every element
        rows, cols = 1, q.numel()
    if k.numel() != rows:
        raise ValueError(f"dequantize: {k.numel()} exponents for {rows} rows")
    out = torch.empty(q.shape, dtype=dtype, device=q.device)
    L = _lib.load()
    _lib.check(
        L.ely_fp8_dequantize(q.data_ptr(), k.data_ptr(), rows, cols, _lib.FMT[fmt], out.data_ptr(), _lib.dtype_code(out), _lib.stream_ptr(q.device)),
        "dequantize",
    )
    return out


def roundtrip(x: torch.Tensor, fmt: str = "e4m3", per_tensor: bool = False, k_hint: int | torch.Tensor | None = None) -> torch.Tensor:
    """The declared recipe at a boundary: quantize then dequantize, in x's
    dtype (model/fp8.py:56-63), fused into one pass.  k_hint as quantize's."""
    f = _fmt(fmt)
    hint = _hint(k_hint, per_tensor, "roundtrip")
    if hint is not None:
        if x.dim() == 0:
            raise ValueError("roundtrip: a 0-d tensor has no rows")
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        _per_tensor_hint(x, f, hint, None, out, "roundtrip")
        return out
    if per_tensor:
        return roundtrip(x.reshape(1, -1), fmt).reshape(x.shape)
    x, rows, cols = _rows(x, "roundtrip")
    out = torch.empty_like(x)
    L = _lib.load()
    ws = _lib.workspace(x.device, L.ely_fp8_workspace_bytes(rows, cols, _lib.dtype_code(x)))
    _lib.check(
        L.ely_fp8_roundtrip(x.data_ptr(), _lib.dtype_code(x), rows, cols, f, out.data_ptr(), None, None, ws.data_ptr(), ws.numel(), _lib.stream_ptr(x.device)),
        "roundtrip",
    )
    return out


def recover_exp(t: torch.Tensor, fmt: str = "e4m3") -> torch.Tensor:
    """Per-row exponent k making t * 2^-k exactly fp8-representable, from the
    dequantized tensor alone: the first of base + (0, -1, 1, -2, 2) that works
    for the whole row (model/fp8.py:66-93).  Raises ValueError when some row
    has none ("recipe mismatch"), as the reference does.  One device
    synchronization (the bad-row count) per call."""
    f = _fmt(fmt)
    t, rows, cols = _rows(t, "recover_exp")
    k = torch.empty(_k_shape(t), dtype=torch.int32, device=t.device)
    bad = torch.zeros(1, dtype=torch.int64, device=t.device)
    L = _lib.load()
    ws = _lib.workspace(t.device, L.ely_fp8_recover_workspace_bytes(rows))
    _lib.check(
        L.ely_fp8_recover_exp(t.data_ptr(), _lib.dtype_code(t), rows, cols, f, k.data_ptr(), bad.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(t.device)),
        "recover_exp",
    )
    if int(bad.item()):
        raise ValueError("boundary tensor is not scaled-FP8 representable: recipe mismatch")
    return k
