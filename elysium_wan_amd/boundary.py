"""Declared narrowing of a stage-boundary tensor on MI355X: the drop-in for
wantrain's model/gpt.py:284-317 (`narrow` and the `_Boundary` autograd
function), the caller of the fp8 codec at every block input and output.

A scaled fp8 format narrows through the fused quantize -> dequantize kernel
(fp8.roundtrip, one HBM read and one write per element); any other declared
dtype is a plain cast there and back, as in the reference.
"""

from __future__ import annotations

import torch

from . import fp8


def narrow(x: torch.Tensor, dtype, needs_scale: bool) -> torch.Tensor:
    """model/gpt.py:284-297: x narrowed to `dtype` and back, in x's dtype.
    fp8 formats are power-of-two scaled per row (last dim)."""
    if dtype is None:
        return x
    if needs_scale:
        return fp8.roundtrip(x, "e5m2" if dtype is torch.float8_e5m2 else "e4m3")
    return x.to(dtype).to(x.dtype)


class Boundary(torch.autograd.Function):
    """model/gpt.py:300-317: forward narrows the activation, backward narrows
    the gradient, with the same format both ways."""

    @staticmethod
    def forward(ctx, x, dtype, needs_scale):
        ctx.dtype, ctx.needs_scale = dtype, needs_scale
        return narrow(x, dtype, needs_scale)

    @staticmethod
    def backward(ctx, g):
        return narrow(g, ctx.dtype, ctx.needs_scale), None, None


def boundary(x: torch.Tensor, dtype, needs_scale: bool) -> torch.Tensor:
    """Boundary.apply with the reference's argument order."""
    return Boundary.apply(x, dtype, needs_scale)
