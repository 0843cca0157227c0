"""The lossless wire codecs of a stage boundary on MI355X: the drop-in for
wantrain's codec/planes.py (encode, decode, encode_scaled_fp8 and the wire
ids).  The byte work runs on the GPU -- the byte-plane split and join, the
scaled-fp8 exponent recovery, byte image and dequantization -- and only the
planes cross PCIe, to be compressed on the host.

Plain dtypes (codec/planes.py:141-190): header "<BBQ" (dtype id, plane
count, element count), one "<I" compressed size per plane, then the planes;
multi-byte elements travel as byte planes, most significant byte first,
single-byte elements interleaved.

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
import os
import struct
import threading
import zlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from . import _lib
from . import fp8 as _fp8

_ZSTD_MAGIC = b"\x28\xb5\x2f\xfd"
# wire dtype ids; append only, never renumber (codec/planes.py:63-70)
_DT = {
    0: torch.float32,
    1: torch.bfloat16,
    2: torch.float16,
    3: torch.float8_e4m3fn,
    4: torch.float8_e5m2,
    5: torch.int64,
}
_ID = {v: k for k, v in _DT.items()}
_HDR = struct.Struct("<BBQ")  # dtype id, plane count, element count
# Scaled-fp8 wire ids live above the plain dtype ids; append only (codec/planes.py:137-138).
_SCALED_ID = {"e4m3": 32, "e5m2": 33}
_SCALED_FMT = {v: k for k, v in _SCALED_ID.items()}


def _compress(b) -> bytes:
    return zlib.compress(b, 1)


_POOL = None
_POOL_PID = None
_POOL_LOCK = threading.Lock()


def _compress_all(bufs) -> list:
    """Each buffer compressed on its own (zlib level 1), the payload's blobs
    in order: the same bytes as one after the other, but the planes go
    through zlib on host threads at once (zlib releases the GIL), so the
    host half of an encode takes its slowest plane's time, not their sum.
    A forked child starts its own pool: the parent's threads do not exist
    there."""
    global _POOL, _POOL_PID
    if len(bufs) < 2 or sum(memoryview(b).nbytes for b in bufs) < (1 << 20):
        return [_compress(b) for b in bufs]
    with _POOL_LOCK:
        if _POOL is None or _POOL_PID != os.getpid():
            _POOL = ThreadPoolExecutor(max_workers=8, thread_name_prefix="ely-planes")
            _POOL_PID = os.getpid()
        pool = _POOL
    return list(pool.map(_compress, bufs))


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
    t = _lib.to_gpu(t, "encode_scaled_fp8")
    t = t.detach().contiguous()
    flat = t.reshape(-1, t.shape[-1]) if t.dim() > 1 else t.reshape(1, -1)
    rows, cols = flat.shape
    # recover_exp's k and the byte image in one device call (fp8.py:66-93, planes.py:110-111)
    k = torch.empty(rows, dtype=torch.int32, device=flat.device)
    q = torch.empty(flat.shape, dtype=torch.uint8, device=flat.device)
    bad = torch.zeros(1, dtype=torch.int64, device=flat.device)
    L = _lib.load()
    ws = _lib.workspace(flat.device, L.ely_fp8_recover_workspace_bytes(rows))
    _lib.check(
        L.ely_fp8_recover_image(flat.data_ptr(), _lib.dtype_code(flat), rows, cols, _lib.FMT[fmt], k.data_ptr(), q.data_ptr(),
                                bad.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(flat.device)),
        "encode_scaled_fp8",
    )
    if int(bad.item()):
        # the reference's recover_exp raises first, with its own message
        # (model/fp8.py:91-92); its later round-trip check (planes.py:104-109)
        # cannot fail once every row has an exact k
        raise ValueError("boundary tensor is not scaled-FP8 representable: recipe mismatch")
    raw = q.reshape(-1).cpu().numpy()
    exps = k.reshape(-1).cpu().numpy().astype(np.int8)  # torch's .to(int8): two's-complement wrap
    c_v = _compress(raw.tobytes())
    c_k = _compress(exps.view(np.uint8).tobytes())
    head = _HDR.pack(_SCALED_ID[fmt], 2, raw.size)
    head += struct.pack("<I", len(c_v)) + struct.pack("<I", len(c_k))
    return head + c_v + c_k, tuple(t.shape)


def encode(t: torch.Tensor):
    """codec/planes.py:141-160: a tensor in its declared boundary dtype ->
    (payload, shape), lossless.  The byte planes are split on the GPU."""
    if t.dtype not in _ID:
        raise ValueError(f"no wire encoding for dtype {t.dtype}")
    t = _lib.to_gpu(t, "encode")
    t = t.detach().contiguous()
    esz = t.element_size()
    n = t.numel()
    raw = t.reshape(-1).view(torch.uint8)
    if esz == 1:
        blobs = [_compress(raw.cpu().numpy().tobytes())]
    else:
        planes = torch.empty(esz * n, dtype=torch.uint8, device=t.device)
        L = _lib.load()
        _lib.check(L.ely_byteplanes_split(raw.data_ptr(), n, esz, planes.data_ptr(), _lib.stream_ptr(t.device)), "encode")
        host = planes.cpu().numpy()
        blobs = _compress_all([host[j * n : (j + 1) * n] for j in range(esz)])
    head = _HDR.pack(_ID[t.dtype], len(blobs), n)
    head += b"".join(struct.pack("<I", len(b)) for b in blobs)
    return head + b"".join(blobs), tuple(t.shape)


def _device(device):
    return torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)


def decode(payload: bytes, shape, device=None) -> torch.Tensor:
    """codec/planes.py:163-190: payload -> tensor of `shape` on `device`
    (default the current CUDA device), bit-identical to what was encoded.
    Scaled-fp8 payloads decode to float32 (codec/planes.py:120-133)."""
    did, nplanes, n = _HDR.unpack_from(payload, 0)
    if did in _SCALED_FMT:
        return _decode_scaled(payload, shape, device)
    if did not in _DT:
        raise ValueError(f"unknown wire dtype id {did}")
    off = _HDR.size
    sizes = []
    for _ in range(nplanes):
        sizes.append(struct.unpack_from("<I", payload, off)[0])
        off += 4
    dtype = _DT[did]
    esz = torch.empty(0, dtype=dtype).element_size()
    if math.prod(shape) != n:
        raise ValueError(f"shape {tuple(shape)} does not hold {n} elements")
    planes = []
    for sz in sizes:
        planes.append(_decompress(payload[off : off + sz]))
        off += sz
    dev = _device(device)
    if nplanes == 1:
        if len(planes[0]) != n * esz:
            raise ValueError(f"payload holds {len(planes[0])} bytes, header says {n * esz}")
        buf = torch.frombuffer(bytearray(planes[0]), dtype=torch.uint8).to(dev) if n else torch.empty(0, dtype=torch.uint8, device=dev)
        return buf.view(dtype).reshape(shape)
    if nplanes != esz or any(len(p) != n for p in planes):
        raise ValueError(f"{nplanes} planes of sizes {[len(p) for p in planes]} do not hold {n} elements of {esz} bytes")
    out = torch.empty(n * esz, dtype=torch.uint8, device=dev)
    if n:
        src = torch.frombuffer(bytearray(b"".join(planes)), dtype=torch.uint8).to(dev)
        L = _lib.load()
        with torch.cuda.device(dev):
            _lib.check(L.ely_byteplanes_join(src.data_ptr(), n, esz, out.data_ptr(), _lib.stream_ptr(dev)), "decode")
    return out.view(dtype).reshape(shape)


def _decode_scaled(payload: bytes, shape, device=None) -> torch.Tensor:
    """codec/planes.py:120-133: a scaled-fp8 payload -> float32 tensor of
    `shape` on `device`, dequantized on the GPU."""
    did, nplanes, n = _HDR.unpack_from(payload, 0)
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
    dev = _device(device)
    q = torch.from_numpy(raw.copy()).to(dev).view(_fp8.FORMATS[fmt][0]).reshape(rows, n // rows)
    k = torch.from_numpy(exps.astype(np.int32)).to(dev).reshape(rows, 1)
    return _fp8.dequantize(q, k, torch.float32).reshape(shape)
