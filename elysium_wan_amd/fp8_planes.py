"""The unscaled e4m3 wire codec with nibble planes on MI355X: the drop-in for
wantrain's codec/fp8_planes.py (encode, decode; same payload bytes and
assertion).

Valid only for a boundary tensor that is exactly representable in
float8_e4m3fn.  One GPU pass converts every element, checks that the code
converts back to it, and splits the codes into a high-nibble and a
low-nibble plane (two nibbles per byte, element 2i in the high half); the
planes are compressed on the host.  Payload: struct "<QII" (element count,
compressed sizes of the two planes), then the two compressed planes.
"""

from __future__ import annotations

import math
import struct

import numpy as np
import torch

from . import _lib
from .planes import _compress_all, _decompress

_HDR = struct.Struct("<QII")


def encode(t: torch.Tensor):
    """codec/fp8_planes.py:19-32: -> (payload, shape).  AssertionError
    "boundary is not FP8-representable: recipe mismatch" when some element
    is not exactly an e4m3 value (NaN never is; -0 counts as 0)."""
    t = _lib.to_gpu(t, "fp8_planes.encode")
    t = t.detach().contiguous()
    if t.dtype not in (torch.float32, torch.bfloat16):
        if not t.is_floating_point():
            raise TypeError(f"fp8_planes encodes floating-point tensors, got {t.dtype}")
        t = t.float()  # float16 and fp8 widen to fp32 exactly
    n = t.numel()
    nb = (n + 1) // 2
    hi = torch.empty(nb, dtype=torch.uint8, device=t.device)
    lo = torch.empty(nb, dtype=torch.uint8, device=t.device)
    bad = torch.zeros(1, dtype=torch.int64, device=t.device)
    L = _lib.load()
    _lib.check(
        L.ely_fp8_nibbles_encode(t.data_ptr(), _lib.dtype_code(t), n, hi.data_ptr(), lo.data_ptr(), bad.data_ptr(), _lib.stream_ptr(t.device)),
        "fp8_planes.encode",
    )
    if int(bad.item()):
        raise AssertionError("boundary is not FP8-representable: recipe mismatch")
    c_hi, c_lo = _compress_all([hi.cpu().numpy(), lo.cpu().numpy()])
    return _HDR.pack(n, len(c_hi), len(c_lo)) + c_hi + c_lo, tuple(t.shape)


def decode(payload: bytes, shape, device=None) -> torch.Tensor:
    """codec/fp8_planes.py:35-52: payload -> float32 tensor of `shape` on
    `device` (default the current CUDA device)."""
    n, nhi, nlo = _HDR.unpack_from(payload, 0)
    off = _HDR.size
    hi = _decompress(payload[off : off + nhi])
    lo = _decompress(payload[off + nhi : off + nhi + nlo])
    nb = (n + 1) // 2
    if len(hi) < nb or len(lo) < nb:
        raise ValueError(f"nibble planes of {len(hi)} and {len(lo)} bytes do not hold {n} codes")
    if math.prod(shape) != n:
        raise ValueError(f"shape {tuple(shape)} does not hold {n} elements")
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    out = torch.empty(n, dtype=torch.float32, device=dev)
    if n:
        h = torch.from_numpy(np.frombuffer(hi, dtype=np.uint8, count=nb).copy()).to(dev)
        lw = torch.from_numpy(np.frombuffer(lo, dtype=np.uint8, count=nb).copy()).to(dev)
        L = _lib.load()
        with torch.cuda.device(dev):
            _lib.check(L.ely_fp8_nibbles_decode(h.data_ptr(), lw.data_ptr(), n, out.data_ptr(), _lib.stream_ptr(dev)), "fp8_planes.decode")
    return out.reshape(shape)
