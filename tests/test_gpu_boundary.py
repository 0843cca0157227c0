"""The codec's caller, model/gpt.py:284-317 (narrow, _Boundary), on the GPU:
forward narrows the activation and backward the gradient with the same
format, bit for bit against the oracle's quantize -> dequantize."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import activation, bits, say

pytestmark = pytest.mark.gpu


def _oracle_roundtrip(oracle, x: torch.Tensor, fmt: str) -> np.ndarray:
    q, k = oracle.quantize(bits(x).reshape(-1, x.shape[-1]), fmt)
    return oracle.dequantize(q, k, fmt, "bf16")


@pytest.mark.parametrize("dtype,fmt", [(torch.float8_e4m3fn, "e4m3"), (torch.float8_e5m2, "e5m2")])
def test_boundary_narrows_both_directions(oracle, dtype, fmt):
    from elysium_wan_amd import boundary

    x = activation((2, 128, 768), seed=31).requires_grad_(True)
    g = activation((2, 128, 768), seed=32, outlier_frac=0) * 1e-5
    say("boundary", fmt)
    y = boundary.boundary(x, dtype, True)
    y.backward(g)
    assert y.dtype == torch.bfloat16 and x.grad.dtype == torch.bfloat16
    assert np.array_equal(bits(y).reshape(-1), _oracle_roundtrip(oracle, x.detach(), fmt).reshape(-1))
    assert np.array_equal(bits(x.grad).reshape(-1), _oracle_roundtrip(oracle, g, fmt).reshape(-1))
    # gradients at 1e-5 survive: the per-row scale keeps them off fp8's zero
    assert float(x.grad.float().abs().sum()) > 0


def test_unscaled_narrowing_is_a_cast_and_none_is_identity():
    from elysium_wan_amd import boundary

    x = torch.randn(4, 64, device="cuda")
    assert boundary.narrow(x, None, False) is x
    assert torch.equal(boundary.narrow(x, torch.bfloat16, False), x.to(torch.bfloat16).float())
