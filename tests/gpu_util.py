"""Helpers shared by the GPU parity tests (numpy views of device tensors,
ulp distances, seeded synthetic inputs)."""

from __future__ import annotations

import sys

import numpy as np
import torch


def say(*a) -> None:
    """Name the case before a GPU step, flushed, so a failed run shows it."""
    print(*a, flush=True)
    sys.stdout.flush()


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bits of a tensor on any device as a numpy array (bf16 -> uint16,
    fp8 -> uint8, fp32 -> float32)."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return t.view(torch.uint8).numpy()
    return t.numpy()


def from_bits_bf16(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16).copy()).view(torch.bfloat16).to(device)


def f32_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise fp32 equality with every NaN equal to every NaN."""
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|ordinal(a) - ordinal(b)| of fp32 values (0 = bit-identical)."""
    ia = a.astype(np.float32).view(np.int32).astype(np.int64)
    ib = b.astype(np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def activation(shape, seed: int, dtype=torch.bfloat16, outlier_frac=1e-3, outlier_scale=50.0, device="cuda"):
    """N(0,1) with a seeded fraction of elements scaled (the benchmark
    configs' activation recipe), generated on the CPU so the bytes are reproducible."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    n = x.numel()
    k = max(1, int(n * outlier_frac)) if outlier_frac > 0 else 0
    if k:
        idx = torch.randperm(n, generator=g)[:k]
        x.view(-1)[idx] *= outlier_scale
    return x.to(dtype).to(device)


def gpt_block_shapes(d: int):
    """The 12 tensors of one GPT block at width d (12 d^2 + 13 d elements):
    ln1 w/b, qkv w/b, proj w/b, ln2 w/b, fc1 w/b, fc2 w/b."""
    return [(d,), (d,), (3 * d, d), (3 * d,), (d, d), (d,), (d,), (d,), (4 * d, d), (4 * d,), (d, 4 * d), (d,)]
