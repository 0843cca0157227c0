"""The scaled-fp8 wire codec of a stage boundary on MI355X: the drop-in for
wantrain's codec/planes.py:85-138 (encode_scaled_fp8, decode and the wire
ids), with the exponent recovery, the byte image and the dequantization on
the GPU.  Only the compressed bytes cross to the host.

Payload layout, unchanged (codec/planes.py:115-117): struct "<BBQ" (wire id
32 for e4m3 / 33 for e5m2, plane count 2, element count), "<I" length of the
compressed fp8 bytes, "<I" length of the compressed int8 exponents, then the
two compressed blobs.  Compression is zlib level 1 -- the reference's own
fallback when the zstandard module is absent (codec/planes.py:23-49), as it
is on these boxes; decode sniffs the zstd magic and refuses it with the
reference's message.
"""

from __future__ import annotations

import math
import struct
import zlib

import numpy as np
import torch

from . import _lib
from . import fp8 as _fp8

_ZSTD_MAGIC = b"\x28\xb5\x2f\xfd"
_HDR = struct.Struct("<BBQ")  # dtype id, plane count, element count
# Scaled-fp8 wire ids live above the plain dtype ids; append only (codec/planes.py:137-138).
_SCALED_ID = {"e4m3": 32, "e5m2": 33}
_SCALED_FMT = {v: k for k, v in _SCALED_ID.items()}


def _compress(b: bytes) -> bytes:
    return zlib.compress(b, 1)


def _decompress(b: bytes) -> bytes:
    if b[:4] == _ZSTD_MAGIC:
        raise RuntimeError(
            "payload is zstd-compressed but the zstandard module is not "
            "installed on this box; the bootstrap must install it"
        )
    return zlib.decompress(b)


def encode_scaled_fp8(t: torch.Tensor, fmt: str = "e4m3"):
    """codec/planes.py:85-117: a boundary tensor that is its own scaled-fp8
    round trip -> (payload bytes, shape).  Rows are the last dim (a 1-d tensor
    is one row); each row's exponent is recovered from the tensor itself and
    the tensor must be exactly representable with it, else ValueError."""
    if fmt not in _SCALED_ID:
        raise ValueError(f"fp8 format {fmt!r} is not one of {tuple(_SCALED_ID)}")
    _lib.require_gpu(t, "encode_scaled_fp8")
    t = t.detach().contiguous()
    flat = t.reshape(-1, t.shape[-1]) if t.dim() > 1 else t.reshape(1, -1)
    try:
        k = _fp8.recover_exp(flat, fmt)  # (rows, 1) int32
    except ValueError:
        raise ValueError(
            "boundary is not scaled-FP8 representable: recipe mismatch. The tensor "
            "reaching the wire must be the recipe's own fp8 round trip."
        ) from None
    rows, cols = flat.shape
    q = torch.empty(flat.shape, dtype=torch.uint8, device=flat.device)
    L = _lib.load()
    _lib.check(
        L.ely_fp8_quantize_k(flat.data_ptr(), _lib.dtype_code(flat), rows, cols, _lib.FMT[fmt], k.data_ptr(), q.data_ptr(), _lib.stream_ptr(flat.device)),
        "encode_scaled_fp8",
    )
    raw = q.reshape(-1).cpu().numpy()
    exps = k.reshape(-1).cpu().numpy().astype(np.int8)  # torch's .to(int8): two's-complement wrap
    c_v = _compress(raw.tobytes())
    c_k = _compress(exps.view(np.uint8).tobytes())
    head = _HDR.pack(_SCALED_ID[fmt], 2, raw.size)
    head += struct.pack("<I", len(c_v)) + struct.pack("<I", len(c_k))
    return head + c_v + c_k, tuple(t.shape)


def decode(payload: bytes, shape, device=None) -> torch.Tensor:
    """codec/planes.py:141-190 for the scaled-fp8 ids: payload -> float32
    tensor of `shape` (on `device`, default the current CUDA device),
    dequantized on the GPU.  Plain-dtype byte-plane payloads are not part of
    this build."""
    did, nplanes, n = _HDR.unpack_from(payload, 0)
    if did not in _SCALED_FMT:
        raise ValueError(f"wire id {did} is not a scaled-fp8 payload (ids {sorted(_SCALED_FMT)})")
    off = _HDR.size
    sizes = []
    for _ in range(nplanes):
        sizes.append(struct.unpack_from("<I", payload, off)[0])
        off += 4
    fmt = _SCALED_FMT[did]
    raw = np.frombuffer(_decompress(payload[off : off + sizes[0]]), dtype=np.uint8)
    off += sizes[0]
    exps = np.frombuffer(_decompress(payload[off : off + sizes[1]]), dtype=np.int8)
    if raw.size != n:
        raise ValueError(f"payload holds {raw.size} fp8 bytes, header says {n}")
    rows = exps.size
    if rows == 0 or n % rows:
        raise ValueError(f"{n} elements do not split into {rows} rows")
    if math.prod(shape) != n:
        raise ValueError(f"shape {tuple(shape)} does not hold {n} elements")
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    q = torch.from_numpy(raw.copy()).to(dev).view(_fp8.FORMATS[fmt][0]).reshape(rows, n // rows)
    k = torch.from_numpy(exps.astype(np.int32)).to(dev).reshape(rows, 1)
    return _fp8.dequantize(q, k, torch.float32).reshape(shape)
