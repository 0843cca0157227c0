"""ctypes binding of libelyhip.so (the C ABI declared in include/ely.h).

There is no fallback: if the library is missing or a GPU call fails, the
caller gets an exception.  Status codes map to the reference's Python errors:
ELY_EINVAL / ELY_ENOTREPR -> ValueError, everything else -> RuntimeError,
both carrying ely_last_error().
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libelyhip.so")

OK, EINVAL, EHIP, ENOTREPR, EWORKSPACE = 0, 1, 2, 3, 4
F32, BF16 = 0, 1
E4M3, E5M2 = 0, 1
ORDER_HOST, ORDER_TORCH = 0, 1
FMT = {"e4m3": E4M3, "e5m2": E5M2}

EXPORTS = (
    "ely_abi_version",
    "ely_last_error",
    "ely_grad_norm_workspace_bytes",
    "ely_grad_norm_clip",
    "ely_grad_norm",
    "ely_grad_norm_fold",
    "ely_adamw_workspace_bytes",
    "ely_adamw_step",
    "ely_adamw_fold_step",
    "ely_fp8_workspace_bytes",
    "ely_fp8_quantize",
    "ely_fp8_quantize_noalloc",
    "ely_fp8_hint_workspace_bytes",
    "ely_fp8_quantize_hint",
    "ely_fp8_dequantize",
    "ely_fp8_roundtrip",
    "ely_fp8_recover_workspace_bytes",
    "ely_fp8_recover_exp",
    "ely_fp8_recover_image",
    "ely_fp8_quantize_k",
    "ely_cast_bf16",
    "ely_fold_add",
    "ely_fold_add_bf16",
    "ely_scale_inplace",
    "ely_rows_fold",
    "ely_rows_split",
    "ely_widen_bf16",
    "ely_set_max_blocks",
    "ely_host_device_pointer",
    "ely_byteplanes_split",
    "ely_byteplanes_join",
    "ely_fp8_nibbles_encode",
    "ely_fp8_nibbles_decode",
    "ely_selftest_fp8_cvt",
    "ely_selftest_fp8_scaled",
    "ely_selftest_sqrt",
)


class ElyTensor(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("numel", ctypes.c_int64), ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class ElyConsts(ctypes.Structure):
    _fields_ = [("c", ctypes.c_float * 8)]


class ElyNormResult(ctypes.Structure):
    _fields_ = [("sumsq", ctypes.c_double), ("norm", ctypes.c_float), ("coef", ctypes.c_float)]


_lib = None
_lock = threading.Lock()


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build the HIP library first "
                "(python -m elysium_wan_amd.build, or __graft_entry__.build())"
            )
        L = ctypes.CDLL(path)
        P, I32, I64, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        TP = ctypes.POINTER(ElyTensor)
        L.ely_abi_version.restype = I32
        L.ely_last_error.restype = ctypes.c_char_p
        L.ely_grad_norm_workspace_bytes.restype = I64
        L.ely_grad_norm_workspace_bytes.argtypes = [TP, I32]
        L.ely_grad_norm.argtypes = [TP, I32, F, P, P, I64, P]
        L.ely_grad_norm_clip.argtypes = [TP, I32, F, P, P, I64, P]
        L.ely_grad_norm_fold.argtypes = [TP, TP, I32, F, P, P, I64, P]
        L.ely_adamw_workspace_bytes.restype = I64
        L.ely_adamw_workspace_bytes.argtypes = [I32]
        L.ely_adamw_step.argtypes = [TP, TP, TP, TP, TP, I32, ctypes.POINTER(ElyConsts), I32, I32, P, P, I64, P]
        L.ely_adamw_fold_step.argtypes = [TP, TP, TP, TP, TP, TP, I32, ctypes.POINTER(ElyConsts), I32, I32, P, P, I64, P]
        L.ely_fp8_workspace_bytes.restype = I64
        L.ely_fp8_workspace_bytes.argtypes = [I64, I64, I32]
        L.ely_fp8_quantize.argtypes = [P, I32, I64, I64, I32, P, P, P, I64, P]
        L.ely_fp8_quantize_noalloc.argtypes = [P, I32, I64, I64, I32, P, P, P]
        L.ely_fp8_hint_workspace_bytes.restype = I64
        L.ely_fp8_hint_workspace_bytes.argtypes = [I64]
        L.ely_fp8_quantize_hint.argtypes = [P, I32, I64, I32, I32, P, P, P, P, P, P, I64, P]
        L.ely_fp8_dequantize.argtypes = [P, P, I64, I64, I32, P, I32, P]
        L.ely_fp8_roundtrip.argtypes = [P, I32, I64, I64, I32, P, P, P, P, I64, P]
        L.ely_fp8_recover_workspace_bytes.restype = I64
        L.ely_fp8_recover_workspace_bytes.argtypes = [I64]
        L.ely_fp8_recover_exp.argtypes = [P, I32, I64, I64, I32, P, P, P, I64, P]
        L.ely_fp8_recover_image.argtypes = [P, I32, I64, I64, I32, P, P, P, P, I64, P]
        L.ely_fp8_quantize_k.argtypes = [P, I32, I64, I64, I32, P, P, P]
        L.ely_cast_bf16.argtypes = [P, P, I64, P]
        L.ely_fold_add.argtypes = [P, P, I32, I64, P]
        L.ely_fold_add_bf16.argtypes = [P, P, I32, I64, P]
        L.ely_scale_inplace.argtypes = [TP, I32, P, P]
        L.ely_rows_fold.argtypes = [P, P, P, P, P, P, I64, I64, I64, I64, I64, I32, I32, P]
        L.ely_rows_split.argtypes = [P, P, P, P, I64, I64, I64, I32, I32, P]
        L.ely_widen_bf16.argtypes = [P, P, I64, P]
        L.ely_set_max_blocks.argtypes = [I32]
        L.ely_host_device_pointer.argtypes = [P, ctypes.POINTER(ctypes.c_void_p)]
        L.ely_byteplanes_split.argtypes = [P, I64, I32, P, P]
        L.ely_byteplanes_join.argtypes = [P, I64, I32, P, P]
        L.ely_fp8_nibbles_encode.argtypes = [P, I32, I64, P, P, P, P]
        L.ely_fp8_nibbles_decode.argtypes = [P, P, I64, P, P]
        L.ely_selftest_fp8_cvt.argtypes = [ctypes.c_uint32, ctypes.c_uint64, I32, P, P]
        L.ely_selftest_fp8_scaled.argtypes = [I32, P, P]
        L.ely_selftest_sqrt.argtypes = [ctypes.c_uint32, ctypes.c_uint64, P, P]
        _lib = L
    return _lib


def check(status: int, what: str) -> None:
    if status == OK:
        return
    msg = load().ely_last_error().decode(errors="replace")
    if status in (EINVAL, ENOTREPR):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (status {status}): {msg}")


# ------------------------------------------------------------------ tensors


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    raise TypeError(f"elysium_wan_amd kernels take float32 or bfloat16 tensors, got {t.dtype}")


def require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what}: the MI355X path runs on the GPU, got a {t.device.type} tensor")


def to_gpu(t: torch.Tensor, what: str) -> torch.Tensor:
    """A wire encoder's input on the GPU: the reference's encoders take a
    tensor on any device (they copy it to the host first), so a host tensor
    is copied to the current GPU; with no GPU this raises as require_gpu."""
    if t.device.type != "cuda" and torch.cuda.is_available():
        return t.to(torch.device("cuda", torch.cuda.current_device()))
    require_gpu(t, what)
    return t


def ely_tensor(t: torch.Tensor | None, dtype: int | None = None) -> ElyTensor:
    if t is None:
        return ElyTensor(None, 0, F32 if dtype is None else dtype, 0)
    return ElyTensor(t.data_ptr() or None, t.numel(), dtype_code(t) if dtype is None else dtype, 0)


_TENSOR_NP = np.dtype([("ptr", "<u8"), ("numel", "<i8"), ("dtype", "<i4"), ("reserved", "<i4")])
_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16}


def tensor_array(ts) -> ctypes.Array:
    """An ely_tensor[] over torch tensors (or ElyTensor entries), built
    column-wise in numpy: a step over a few hundred tensors spends tens of
    microseconds here, not milliseconds."""
    n = len(ts)
    table = np.zeros(max(1, n), dtype=_TENSOR_NP)
    if n:
        if any(isinstance(t, ElyTensor) for t in ts):
            for i, t in enumerate(ts):
                e = t if isinstance(t, ElyTensor) else ely_tensor(t)
                table[i] = (e.ptr or 0, e.numel, e.dtype, 0)
        else:
            try:
                table["dtype"][:n] = [_DTYPE_CODE[t.dtype] for t in ts]
            except KeyError:
                for t in ts:
                    dtype_code(t)  # raises the TypeError naming the dtype
            table["ptr"][:n] = [t.data_ptr() for t in ts]
            table["numel"][:n] = [t.numel() for t in ts]
    return (ElyTensor * max(1, n)).from_buffer(table)


def host_device_pointer(t: torch.Tensor) -> int | None:
    """The address under which the GPU reaches the pinned host tensor `t`
    in place (ely_host_device_pointer), or None when it cannot."""
    L = load()
    d = ctypes.c_void_p()
    if L.ely_host_device_pointer(t.data_ptr(), ctypes.byref(d)) != OK or not d.value:
        return None
    return d.value


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# ---------------------------------------------------------------- workspace

_ws: dict = {}
_ws_lock = threading.Lock()


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A scratch byte buffer of at least nbytes, one per (device, current
    stream).  Calls on one stream are ordered, so reuse is safe; when it
    grows, the old buffer returns to torch's allocator, which reuses it only
    after work already queued on that stream."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    nbytes = max(int(nbytes), 256)
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _ws[key] = buf
        return buf
