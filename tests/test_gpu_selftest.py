"""The hardware facts the kernels rely on, checked over every input:
the gfx950 fp8 conversion instructions equal torch's rounding (restated in
ely_device.hpp) on every fp32 pattern the instruction path can see, the
scaled conversions of the bf16 kernels equal it on every bf16 pattern and
exponent they meet, and the kernels' fp32 sqrt equals the reference's fp64 sqrt rounded to fp32
(runtime/optim.py:288-291) on every non-negative fp32 pattern."""

from __future__ import annotations

import pytest
import torch

from gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_fp8_instruction_equals_restatement_on_every_fp32(fmt):
    from elysium_wan_amd import _lib

    L = _lib.load()
    say("selftest fp8 cvt", fmt)
    cnt = torch.zeros(3, dtype=torch.int64, device="cuda")
    _lib.check(L.ely_selftest_fp8_cvt(0, 1 << 32, _lib.FMT[fmt], cnt.data_ptr(), _lib.stream_ptr(cnt.device)), "selftest")
    c = cnt.cpu().tolist()
    say("  mismatches in domain / outside / decode:", c)
    assert c[0] == 0 and c[2] == 0


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_scaled_conversions_equal_the_restatement_on_every_bf16_and_k(fmt):
    """The bf16 kernels quantize and decode with the scaled instructions at
    scale 2^k: every bf16 pattern x every |k| <= 110 of the instruction
    path's domain quantizes to the restatement's code, and every code that is
    not a NaN decodes to the restatement's bf16."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    say("selftest fp8 scaled", fmt)
    cnt = torch.zeros(2, dtype=torch.int64, device="cuda")
    _lib.check(L.ely_selftest_fp8_scaled(_lib.FMT[fmt], cnt.data_ptr(), _lib.stream_ptr(cnt.device)), "selftest scaled")
    c = cnt.cpu().tolist()
    say("  quantize / decode mismatches:", c)
    assert c == [0, 0]


def test_sqrt_is_the_fp64_sqrt_rounded_once():
    from elysium_wan_amd import _lib

    L = _lib.load()
    say("selftest sqrt")
    cnt = torch.zeros(1, dtype=torch.int64, device="cuda")
    _lib.check(L.ely_selftest_sqrt(0, 1 << 31, cnt.data_ptr(), _lib.stream_ptr(cnt.device)), "selftest sqrt")
    assert int(cnt.item()) == 0
