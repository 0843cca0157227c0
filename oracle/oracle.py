"""CPU oracle for the per-stage update path -- TEST INFRASTRUCTURE ONLY.

The parity checker the HIP kernels are held to.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module; the product package (elysium_wan_amd) never does, and fails loudly
when its HIP library is missing instead of falling back here.

numpy wrappers over the C restatement in ely_oracle.c, plus the two pieces
that are host-side in the reference too:

* `host_adamw_consts` -- HostAdamW.step's per-step fp32 constants
  (runtime/optim.py:149-167 with _f32 at :72-74), computed in double by the
  same Python expressions and rounded once to fp32.
* `torch_adamw_consts` -- the scalars torch's _multi_tensor_adam hands its
  foreach kernels (TORCH/optim/adam.py:689-800).
* `wire_encode` / `wire_decode` -- the scaled-fp8 wire image of
  codec/planes.py:85-133 (header <BBQ>, two <I> sizes, fp8 bytes, int8
  exponents), with zlib level 1, the reference's compressor when zstandard
  is absent (codec/planes.py:23-27, 44-49).

Every function's provenance is in ely_oracle.c's header; the checks that pin
each one against torch, the reference's golden vectors and closed forms are
in tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import math
import os
import struct
import zlib

import numpy as np

DT_F32, DT_BF16 = 0, 1
FMT = {"e4m3": 0, "e5m2": 1}
EBIAS = {"e4m3": 8, "e5m2": 15}
_DELTAS = (0, -1, 1, -2, 2)
SCALED_ID = {"e4m3": 32, "e5m2": 33}

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libely_oracle.so")
_lib = None


def build() -> str:
    """Compile the C restatement with oracle/Makefile (gcc)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "-B", "libely_oracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64, I32, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [F]
        L.orc_f32_to_fp8.restype = ctypes.c_uint8
        L.orc_f32_to_fp8.argtypes = [F, I32]
        L.orc_fp8_encode_array.argtypes = [P, I64, I32, P]
        L.orc_fp8_to_f32.restype = F
        L.orc_fp8_to_f32.argtypes = [ctypes.c_uint8, I32]
        L.orc_pow2.restype = F
        L.orc_pow2.argtypes = [I32, I32]
        L.orc_scale_exp.argtypes = [P, I32, I64, I64, I32, P]
        L.orc_quantize.argtypes = [P, I32, I64, I64, I32, P, P]
        L.orc_dequantize.argtypes = [P, P, I64, I64, I32, P, I32]
        L.orc_recover_exp.restype = I64
        L.orc_recover_exp.argtypes = [P, I32, I64, I64, I32, P]
        for name in ("orc_adamw_host", "orc_adamw_torch"):
            f = getattr(L, name)
            f.argtypes = [P, P, I32, P, P, I64, P, I32, F, P]
        L.orc_sumsq_d.restype = ctypes.c_double
        L.orc_sumsq_d.argtypes = [P, I32, I64]
        L.orc_clip_coef.restype = F
        L.orc_clip_coef.argtypes = [F, F]
        L.orc_cast_bf16.argtypes = [P, P, I64]
        L.orc_fold_add.argtypes = [P, P, I32, I64]
        L.orc_fold_add_bf16.argtypes = [P, P, I32, I64]
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _dt(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return DT_F32
    if a.dtype == np.uint16:  # bf16 bit patterns
        return DT_BF16
    raise TypeError(f"oracle takes float32 or bf16-as-uint16 arrays, got {a.dtype}")


# --------------------------------------------------------------- scalars


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size, dtype=np.uint16)
    lib().orc_cast_bf16(_ptr(x), _ptr(out), x.size)
    return out


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def fp8_encode(x: np.ndarray, fmt: str) -> np.ndarray:
    """fp32 values -> fp8 codes (shape kept)."""
    flat = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(flat.size, dtype=np.uint8)
    lib().orc_fp8_encode_array(_ptr(flat), flat.size, FMT[fmt], _ptr(out))
    return out.reshape(np.shape(x))


def fp8_decode_table(fmt: str) -> np.ndarray:
    L, f = lib(), FMT[fmt]
    return np.array([L.orc_fp8_to_f32(c, f) for c in range(256)], dtype=np.float32)


def pow2(n: int, dtype: int) -> float:
    return lib().orc_pow2(int(n), dtype)


# ------------------------------------------------------------------ fp8


def _rows(x: np.ndarray):
    x = np.ascontiguousarray(x)
    if x.ndim == 0:
        raise ValueError("fp8 rows need at least one dimension")
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    return x, rows, cols


def scale_exp(x: np.ndarray, fmt: str = "e4m3") -> np.ndarray:
    """model/fp8.py:28-38 -> int32 [rows]."""
    x, rows, cols = _rows(x)
    k = np.empty(rows, dtype=np.int32)
    lib().orc_scale_exp(_ptr(x), _dt(x), rows, cols, FMT[fmt], _ptr(k))
    return k


def quantize(x: np.ndarray, fmt: str = "e4m3"):
    """model/fp8.py:45-49 -> (uint8 codes shaped like x, int32 k [rows])."""
    x, rows, cols = _rows(x)
    q = np.empty(x.shape, dtype=np.uint8)
    k = np.empty(rows, dtype=np.int32)
    lib().orc_quantize(_ptr(x), _dt(x), rows, cols, FMT[fmt], _ptr(q), _ptr(k))
    return q, k


def dequantize(q: np.ndarray, k: np.ndarray, fmt: str = "e4m3", out_dtype: str = "f32") -> np.ndarray:
    """model/fp8.py:52-53.  out_dtype "f32" -> float32, "bf16" -> uint16 bits."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    k = np.ascontiguousarray(k, dtype=np.int32).reshape(-1)
    cols = q.shape[-1]
    rows = q.size // cols if cols else 0
    if k.size != rows:
        raise ValueError(f"{k.size} exponents for {rows} rows")
    od = DT_F32 if out_dtype == "f32" else DT_BF16
    out = np.empty(q.shape, dtype=np.float32 if od == DT_F32 else np.uint16)
    lib().orc_dequantize(_ptr(q), _ptr(k), rows, cols, FMT[fmt], _ptr(out), od)
    return out


def roundtrip(x: np.ndarray, fmt: str = "e4m3") -> np.ndarray:
    """model/fp8.py:56-63: dequantize(quantize(x)) in x's own dtype."""
    q, k = quantize(x, fmt)
    return dequantize(q, k, fmt, "f32" if _dt(np.asarray(x)) == DT_F32 else "bf16")


def recover_exp(t: np.ndarray, fmt: str = "e4m3"):
    """model/fp8.py:66-93 -> (int32 k [rows], number of rows with no exact k)."""
    t, rows, cols = _rows(t)
    k = np.empty(rows, dtype=np.int32)
    bad = lib().orc_recover_exp(_ptr(t), _dt(t), rows, cols, FMT[fmt], _ptr(k))
    return k, int(bad)


# ----------------------------------------------------------------- wire


def _flat_rows(t: np.ndarray):
    return t.reshape(-1, t.shape[-1]) if t.ndim > 1 else t.reshape(1, -1)


def wire_encode(t: np.ndarray, fmt: str = "e4m3") -> bytes:
    """codec/planes.py:85-117 (zlib-1 container).  Raises ValueError when the
    tensor is not its own scaled-fp8 round trip."""
    flat = _flat_rows(np.ascontiguousarray(t))
    k, bad = recover_exp(flat, fmt)
    if bad:
        raise ValueError("boundary tensor is not scaled-FP8 representable: recipe mismatch")
    dt = _dt(flat)
    rows, cols = flat.shape
    q = np.empty(flat.shape, dtype=np.uint8)
    for r in range(rows):
        s = pow2(-int(k[r]), dt)
        row = flat[r].astype(np.float32) if dt == DT_F32 else bf16_bits_to_f32(flat[r])
        y = row * np.float32(s)
        if dt == DT_BF16:
            y = bf16_bits_to_f32(f32_to_bf16_bits(y))
        q[r] = fp8_encode(y, fmt)
    raw = q.reshape(-1).tobytes()
    exps = k.astype(np.int8).tobytes()  # torch .to(int8): two's-complement wrap
    c_v = zlib.compress(raw, 1)
    c_k = zlib.compress(exps, 1)
    head = struct.pack("<BBQ", SCALED_ID[fmt], 2, len(raw))
    head += struct.pack("<I", len(c_v)) + struct.pack("<I", len(c_k))
    return head + c_v + c_k


def wire_decode(payload: bytes, shape) -> np.ndarray:
    """codec/planes.py:120-133, 150-158: fp32 out."""
    did, nplanes, n = struct.unpack_from("<BBQ", payload, 0)
    off = struct.calcsize("<BBQ")
    sizes = []
    for _ in range(nplanes):
        sizes.append(struct.unpack_from("<I", payload, off)[0])
        off += 4
    fmt = {v: k for k, v in SCALED_ID.items()}[did]
    raw = np.frombuffer(zlib.decompress(payload[off : off + sizes[0]]), dtype=np.uint8)
    off += sizes[0]
    exps = np.frombuffer(zlib.decompress(payload[off : off + sizes[1]]), dtype=np.int8).astype(np.int32)
    rows = exps.size
    out = dequantize(raw.reshape(rows, -1), exps, fmt, "f32")
    return out.reshape(shape)


# ---------------------------------------------------------------- AdamW


def _f32(x: float) -> float:
    """runtime/optim.py:72-74: a double rounded once to fp32."""
    return float(np.float32(x))


def host_adamw_consts(lr: float, betas, eps: float, weight_decay: float, step: float) -> np.ndarray:
    """runtime/optim.py:158-167 for step t (the already-incremented count)."""
    b1, b2 = betas
    t = float(np.float32(step))
    return np.array(
        [
            _f32(1.0 - lr * weight_decay),
            _f32(b1),
            _f32(1.0 - b1),
            _f32(b2),
            _f32(1.0 - b2),
            _f32(1.0 / math.sqrt(1.0 - b2**t)),
            _f32(eps),
            _f32(lr / (1.0 - b1**t)),
        ],
        dtype=np.float32,
    )


def torch_adamw_consts(lr: float, betas, eps: float, weight_decay: float, step: float) -> np.ndarray:
    """The fp32 scalars of _multi_tensor_adam (TORCH/optim/adam.py:689-800):
    decay, 1-b1, b2, 1-b2, bc2**0.5, eps, (lr/bc1)*-1."""
    b1, b2 = betas
    t = float(np.float32(step))
    bc1 = 1 - b1**t
    bc2 = 1 - b2**t
    return np.array(
        [
            _f32(1 - lr * weight_decay),
            _f32(1 - b1),
            _f32(b2),
            _f32(1 - b2),
            _f32(bc2**0.5),
            _f32(eps),
            _f32((lr / bc1) * -1),
        ],
        dtype=np.float32,
    )


def adamw_host(p, g, m, v, consts, weight_decay_nonzero: bool, coef: float = 1.0, copy=None) -> None:
    """runtime/optim.py:277-298 in place on float32 p, m, v; g float32 or bf16 bits."""
    for a in (p, m, v):
        if a.dtype != np.float32 or not a.flags.c_contiguous:
            raise TypeError("p, m, v must be contiguous float32")
    g = np.ascontiguousarray(g)
    c = np.ascontiguousarray(consts, dtype=np.float32)
    cp = _ptr(copy) if copy is not None else None
    lib().orc_adamw_host(_ptr(p), _ptr(g), _dt(g), _ptr(m), _ptr(v), p.size, _ptr(c), int(bool(weight_decay_nonzero)), float(np.float32(coef)), cp)


def adamw_torch(p, g, m, v, consts, weight_decay_nonzero: bool, coef: float = 1.0, copy=None) -> None:
    g = np.ascontiguousarray(g)
    c = np.ascontiguousarray(consts, dtype=np.float32)
    cp = _ptr(copy) if copy is not None else None
    lib().orc_adamw_torch(_ptr(p), _ptr(g), _dt(g), _ptr(m), _ptr(v), p.size, _ptr(c), int(bool(weight_decay_nonzero)), float(np.float32(coef)), cp)


def sumsq(grads) -> float:
    """Brute-force sum of squares over a list of grads (long double per tensor)."""
    total = 0.0
    L = lib()
    for g in grads:
        g = np.ascontiguousarray(g)
        total += L.orc_sumsq_d(_ptr(g), _dt(g), g.size)
    return total


def clip_coef(total_norm: float, max_norm: float) -> float:
    return lib().orc_clip_coef(float(np.float32(total_norm)), float(np.float32(max_norm)))


def cast_bf16(x: np.ndarray) -> np.ndarray:
    return f32_to_bf16_bits(x).reshape(np.shape(x))


def fold_add(acc: np.ndarray, g: np.ndarray) -> None:
    g = np.ascontiguousarray(g)
    lib().orc_fold_add(_ptr(acc), _ptr(g), _dt(g), acc.size)


def fold_add_bf16(acc: np.ndarray, g: np.ndarray) -> None:
    """runtime/accumulate.py:101-102 on a bf16 sum, in place on acc (bf16
    bits as uint16): acc = bf16(float(acc) + float(g))."""
    if acc.dtype != np.uint16 or not acc.flags.c_contiguous:
        raise TypeError("a bf16 sum is contiguous bf16 bits (uint16)")
    g = np.ascontiguousarray(g)
    lib().orc_fold_add_bf16(_ptr(acc), _ptr(g), _dt(g), acc.size)


# ----------------------------------------------------------- plane codecs

# codec/planes.py:63-70: wire dtype ids and element sizes (torch dtype names).
PLANE_IDS = {"float32": 0, "bfloat16": 1, "float16": 2, "float8_e4m3fn": 3, "float8_e5m2": 4, "int64": 5}
PLANE_ESZ = {0: 4, 1: 2, 2: 2, 3: 1, 4: 1, 5: 8}


def byte_planes(raw: np.ndarray, esz: int) -> list:
    """codec/planes.py:152-158: the little-endian elements of `raw` (bytes,
    esz per element) split into esz planes, most significant byte first; one
    interleaved plane for single-byte elements."""
    b = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, esz)
    if esz == 1:
        return [b.reshape(-1).copy()]
    return [b[:, j].copy() for j in range(esz - 1, -1, -1)]


def planes_encode(raw: np.ndarray, dtype_name: str) -> bytes:
    """codec/planes.py:141-160: header <BBQ> (id, plane count, elements),
    one <I> size per plane, then each plane compressed (zlib-1)."""
    did = PLANE_IDS[dtype_name]
    esz = PLANE_ESZ[did]
    blobs = [zlib.compress(p.tobytes(), 1) for p in byte_planes(raw, esz)]
    head = struct.pack("<BBQ", did, len(blobs), raw.size // esz)
    head += b"".join(struct.pack("<I", len(b)) for b in blobs)
    return head + b"".join(blobs)


def planes_decode(payload: bytes) -> tuple:
    """codec/planes.py:163-190 for the plain ids -> (dtype id, element bytes)."""
    did, nplanes, n = struct.unpack_from("<BBQ", payload, 0)
    off = struct.calcsize("<BBQ")
    sizes = []
    for _ in range(nplanes):
        sizes.append(struct.unpack_from("<I", payload, off)[0])
        off += 4
    esz = PLANE_ESZ[did]
    planes = []
    for sz in sizes:
        planes.append(np.frombuffer(zlib.decompress(payload[off : off + sz]), dtype=np.uint8))
        off += sz
    if nplanes == 1:
        return did, planes[0].copy()
    out = np.empty((n, esz), dtype=np.uint8)
    for i, p in enumerate(planes):
        out[:, esz - 1 - i] = p
    return did, out.reshape(-1)


def f32_planes_encode(raw: np.ndarray) -> bytes:
    """codec/f32_planes.py:17-26: float32 elements (as raw bytes, 4 per
    element) -> <Q> count + zlib-1 of the 4 byte planes, byte 0 (least
    significant) first: planes.py's byte planes in the reverse order."""
    b = np.ascontiguousarray(raw, dtype=np.uint8)
    planes = byte_planes(b, 4)[::-1]
    return struct.pack("<Q", b.size // 4) + zlib.compress(b"".join(p.tobytes() for p in planes), 1)


def f32_planes_decode(payload: bytes) -> np.ndarray:
    """codec/f32_planes.py:29-33 -> the elements' raw bytes."""
    (n,) = struct.unpack_from("<Q", payload, 0)
    planes = np.frombuffer(zlib.decompress(payload[8:]), dtype=np.uint8).reshape(4, n)
    return np.ascontiguousarray(planes.T).reshape(-1)


def nibble_planes(codes: np.ndarray):
    """codec/fp8_planes.py:27-30: each e4m3 code's high and low nibble, two
    nibbles per byte in element order (element 2i in the high half), the last
    byte's low half zero for an odd count."""
    c = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    n = c.size
    hi, lo = c >> 4, c & 0x0F
    if n % 2:
        hi = np.append(hi, np.uint8(0))
        lo = np.append(lo, np.uint8(0))
    return ((hi[0::2] << 4) | hi[1::2]).astype(np.uint8), ((lo[0::2] << 4) | lo[1::2]).astype(np.uint8)


def fp8_planes_encode(t: np.ndarray) -> bytes:
    """codec/fp8_planes.py:19-32: t (float32, or bf16 bits as uint16) must be
    exactly e4m3-representable (AssertionError otherwise, as the reference's
    assert); payload <QII> + zlib(high nibbles) + zlib(low nibbles)."""
    t = np.ascontiguousarray(t)
    x = t.astype(np.float32) if t.dtype == np.float32 else bf16_bits_to_f32(t)
    codes = fp8_encode(x.reshape(-1), "e4m3")
    back = fp8_decode_table("e4m3")[codes]
    if not np.array_equal(back, x.reshape(-1)):  # NaN never equal, -0 == 0 (torch.equal)
        raise AssertionError("boundary is not FP8-representable: recipe mismatch")
    hi_p, lo_p = nibble_planes(codes)
    c_hi, c_lo = zlib.compress(hi_p.tobytes(), 1), zlib.compress(lo_p.tobytes(), 1)
    return struct.pack("<QII", codes.size, len(c_hi), len(c_lo)) + c_hi + c_lo


def fp8_planes_decode(payload: bytes) -> np.ndarray:
    """codec/fp8_planes.py:35-52: -> float32 values."""
    n, nhi, nlo = struct.unpack_from("<QII", payload, 0)
    off = struct.calcsize("<QII")
    hi_p = np.frombuffer(zlib.decompress(payload[off : off + nhi]), dtype=np.uint8)
    lo_p = np.frombuffer(zlib.decompress(payload[off + nhi : off + nhi + nlo]), dtype=np.uint8)
    hi = np.stack([hi_p >> 4, hi_p & 0x0F], axis=1).reshape(-1)[:n]
    lo = np.stack([lo_p >> 4, lo_p & 0x0F], axis=1).reshape(-1)[:n]
    codes = ((hi << 4) | lo).astype(np.uint8)
    return fp8_decode_table("e4m3")[codes]
