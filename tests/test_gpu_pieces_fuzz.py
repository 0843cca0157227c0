"""Property-based fuzz of the stand-alone elementwise passes on the GPU:
pieces.cast_piece, pieces.fold_start, pieces.fold_add and the in-place
scale over random sizes
(quad tails, several grid strides) and element offsets (the vector and the
scalar paths), bit for bit against torch on the GPU -- each is one IEEE
rounding per element (runtime/pieces.py:192-214, clip_grad.py:170-177).
Derandomized."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from gpu_util import say

pytestmark = pytest.mark.gpu

FUZZ = settings(max_examples=40, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])


def _at(x: torch.Tensor, off: int) -> torch.Tensor:
    buf = torch.empty(x.numel() + off, dtype=x.dtype, device="cuda")
    buf[off:] = x
    return buf[off:]


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    it = torch.int16 if a.dtype == torch.bfloat16 else torch.int32
    return torch.equal(a.view(it), b.view(it))


@FUZZ
@given(n=st.integers(0, 3_000_000), offs=st.tuples(st.integers(0, 3), st.integers(0, 3)), bf16g=st.booleans(),
       coef=st.sampled_from([1.0, 0.5, 0.3712, 0.0, -1.25]), seed=st.integers(0, 2**16))
def test_elementwise_passes_match_torch(n, offs, bf16g, coef, seed):
    from elysium_wan_amd import _lib, pieces

    gen = torch.Generator(device="cuda").manual_seed(seed)
    say("pieces fuzz", n, offs, "bf16" if bf16g else "f32", coef)
    x = _at(torch.randn(n, device="cuda", generator=gen) * 3, offs[0])
    got = pieces.cast_piece(x, torch.bfloat16)
    assert _same(got, x.to(torch.bfloat16))
    gdt = torch.bfloat16 if bf16g else torch.float32
    g = _at(torch.randn(n, device="cuda", generator=gen).to(gdt), offs[1])
    acc = _at(torch.randn(n, device="cuda", generator=gen), offs[0])
    want = acc + g.float()
    pieces.fold_add(acc, g)
    assert _same(acc, want)
    gb = g if bf16g else _at(g.to(torch.bfloat16), offs[1])
    assert _same(pieces.fold_start(gb), gb.float())  # the widening kernel, vector and scalar paths
    if n:
        L = _lib.load()
        c = torch.tensor([coef], dtype=torch.float32, device="cuda")
        h = g.clone() if offs[1] == 0 else _at(g.clone(), offs[1])
        want = (h.float() * c).to(gdt)
        _lib.check(L.ely_scale_inplace(_lib.tensor_array([h]), 1, c.data_ptr(), _lib.stream_ptr(h.device)), "scale")
        assert _same(h, want)


@pytest.mark.parametrize("n_t", [1, 48, 49, 130])
def test_scale_over_a_tensor_list_equals_torch(n_t):
    """ely_scale_inplace over a list (one launch per 48 tensors): every
    tensor, bf16 or fp32, aligned or at an odd offset, empty or not, equals
    torch's g * coef rounded to its dtype on the GPU."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    gen = torch.Generator(device="cuda").manual_seed(900 + n_t)
    rng = np.random.default_rng(n_t)
    c = torch.tensor([0.37], dtype=torch.float32, device="cuda")
    hs, wants = [], []
    for j in range(n_t):
        n = int(rng.choice([0, 1, 7, 4096, 4097, 20000]))
        dt = torch.bfloat16 if j % 2 else torch.float32
        h = _at(torch.randn(n, device="cuda", generator=gen).to(dt), int(rng.integers(0, 4)))
        wants.append((h.float() * c).to(dt))
        hs.append(h)
    say("scale over a list", n_t)
    _lib.check(L.ely_scale_inplace(_lib.tensor_array(hs), n_t, c.data_ptr(), _lib.stream_ptr(torch.device("cuda", 0))), "scale")
    for h, w in zip(hs, wants):
        assert _same(h, w)


def test_fold_start_widens_every_bf16_pattern_exactly():
    """pieces.fold_start's bf16 -> fp32 kernel on all 65,536 bf16 bit
    patterns (NaNs, infinities, subnormals and both zeros included), aligned
    and one element off: the fp32 bits are the bf16 bits moved to the top,
    which is also what torch's widening gives."""
    from elysium_wan_amd import pieces

    pats = torch.arange(65536, dtype=torch.int32, device="cuda").to(torch.int16).view(torch.bfloat16)
    want = (pats.view(torch.int16).to(torch.int32) << 16).view(torch.float32)
    for off in (0, 1):
        x = _at(pats, off)
        say("fold_start exhaustive, offset", off)
        got = pieces.fold_start(x)
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))
        assert torch.equal(got.view(torch.int32), x.float().view(torch.int32))
