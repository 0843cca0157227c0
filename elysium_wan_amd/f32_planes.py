"""The fp32 lossless wire (codec/f32_planes.py:17-33): the gradient codec of
the fp8_planes wire when the boundary is not fp8 (runtime/stage.py:1646-1650;
decoded by transport/framing.py:81-83).

A float32 tensor's elements are split into 4 byte planes on the GPU (the
byte-plane kernels of the planes wire), least significant byte first as the
reference orders them, and the planes go out as one compressed blob behind
an <Q> element count.  Decode reverses it on the GPU, bit for bit.  As with
the other wires, decode returns the tensor on the GPU where the reference
returns a CPU tensor."""

from __future__ import annotations

import math
import struct

import numpy as np
import torch

from elysium_wan_amd import _lib
from elysium_wan_amd.planes import _compress, _decompress, _device


def encode(t: torch.Tensor):
    """codec/f32_planes.py:17-26: float32 tensor -> (payload, shape)."""
    assert t.dtype == torch.float32  # the reference's own check (an AssertionError)
    t = _lib.to_gpu(t, "f32_planes.encode")
    t = t.detach().contiguous()
    n = t.numel()
    host = np.empty((4, 0), dtype=np.uint8)
    if n:
        planes = torch.empty(4 * n, dtype=torch.uint8, device=t.device)
        L = _lib.load()
        _lib.check(L.ely_byteplanes_split(t.data_ptr(), n, 4, planes.data_ptr(), _lib.stream_ptr(t.device)), "f32_planes.encode")
        # the kernel writes the most significant plane first; this wire starts at byte 0
        host = planes.cpu().numpy().reshape(4, n)[::-1]
    payload = struct.pack("<Q", n) + _compress(np.ascontiguousarray(host).tobytes())
    return payload, tuple(t.shape)


def decode(payload: bytes, shape, device=None) -> torch.Tensor:
    """codec/f32_planes.py:29-33: payload -> float32 tensor of `shape` on
    `device` (default the current CUDA device)."""
    (n,) = struct.unpack_from("<Q", payload, 0)
    planes = np.frombuffer(_decompress(payload[8:]), dtype=np.uint8)
    if planes.size != 4 * n:
        raise ValueError(f"payload holds {planes.size} plane bytes, header says {4 * n}")
    if math.prod(shape) != n:  # numpy's reshape refuses it in the reference
        raise ValueError(f"cannot reshape {n} elements into shape {tuple(shape)}")
    dev = _device(device)
    out = torch.empty(n, dtype=torch.float32, device=dev)
    if n:
        src = torch.from_numpy(np.ascontiguousarray(planes.reshape(4, n)[::-1]).reshape(-1)).to(dev)
        L = _lib.load()
        with torch.cuda.device(dev):
            _lib.check(L.ely_byteplanes_join(src.data_ptr(), n, 4, out.data_ptr(), _lib.stream_ptr(dev)), "f32_planes.decode")
    return out.reshape(shape)
