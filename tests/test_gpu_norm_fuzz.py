"""Property-based fuzz of the grad-norm and the one-call clip on the GPU:
ragged lists of bf16 and fp32 gradients (mixed in one call or not), sizes
around both tile lengths, views at odd element offsets, several max_norm
values.  The sum of squares is within 1e-6 of the oracle's exact sum and
bitwise the same under a capped grid; the coefficient is the oracle's
(torch's formula); ely_grad_norm_clip leaves every gradient at g * coef
rounded once to its dtype.  Derandomized."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from gpu_util import bits, say

pytestmark = pytest.mark.gpu

FUZZ = settings(max_examples=40, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
SIZES = [0, 1, 7, 511, 512, 4095, 4096, 4097, 16383, 16384, 16385, 100_003]

grad_spec = st.tuples(st.sampled_from(SIZES), st.booleans(), st.sampled_from([0, 0, 1, 3]))


def _run(L, _lib, gs, max_norm, clip):
    dev = gs[0].device
    res = torch.zeros(16, dtype=torch.uint8, device=dev)
    arr = _lib.tensor_array(gs)
    ws = torch.empty(L.ely_grad_norm_workspace_bytes(arr, len(gs)), dtype=torch.uint8, device=dev)
    fn = L.ely_grad_norm_clip if clip else L.ely_grad_norm
    _lib.check(fn(arr, len(gs), float(max_norm), res.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev)), "norm")
    r = res.cpu().numpy()
    return r[:8].view(np.float64)[0], r[8:12].view(np.float32)[0], r[12:16].view(np.float32)[0]


@FUZZ
@given(specs=st.lists(grad_spec, min_size=1, max_size=8), max_norm=st.sampled_from([1.0, 1e-3, 0.0, 50.0]), seed=st.integers(0, 2**16))
def test_norm_and_clip_match_the_oracle(oracle, specs, max_norm, seed):
    from elysium_wan_amd import _lib

    L = _lib.load()
    rng = np.random.default_rng(seed)
    gs, host = [], []
    for n, is_bf16, off in specs:
        x = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 4))).astype(np.float32)
        if is_bf16:
            h = oracle.f32_to_bf16_bits(x)
            buf = torch.zeros(n + off, dtype=torch.bfloat16, device="cuda")
            buf[off:] = torch.from_numpy(h.view(np.int16).copy()).view(torch.bfloat16).cuda()
        else:
            h = x
            buf = torch.zeros(n + off, dtype=torch.float32, device="cuda")
            buf[off:] = torch.from_numpy(x).cuda()
        gs.append(buf[off:])
        host.append(h)
    if sum(g.numel() for g in gs) == 0:
        return
    say("norm fuzz", [(n, b, o) for n, b, o in specs], max_norm, seed)
    exact = oracle.sumsq(host)
    s0, norm, coef = _run(L, _lib, gs, max_norm, clip=False)
    assert abs(s0 - exact) <= 1e-6 * exact or (exact == 0.0 and s0 == 0.0)
    assert coef == np.float32(oracle.clip_coef(float(norm), max_norm))
    L.ely_set_max_blocks(7)
    try:
        s1, _, _ = _run(L, _lib, gs, max_norm, clip=False)
    finally:
        L.ely_set_max_blocks(0)
    assert np.float64(s1).view(np.uint64) == np.float64(s0).view(np.uint64)
    s2, _, c2 = _run(L, _lib, gs, max_norm, clip=True)
    assert np.float64(s2).view(np.uint64) == np.float64(s0).view(np.uint64) and c2 == coef
    for g, h in zip(gs, host):
        if g.dtype == torch.bfloat16:
            want = oracle.f32_to_bf16_bits(oracle.bf16_bits_to_f32(h) * np.float32(coef))
            assert np.array_equal(bits(g), want)
        else:
            assert np.array_equal(bits(g).view(np.uint32), (h * np.float32(coef)).astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("n_t", [48, 49])
def test_fold_norm_either_side_of_the_argument_table_limit(oracle, n_t):
    """ely_grad_norm_fold (the sum of squares of acc + widen(g)) with 48
    descriptors by argument and 49 from the uploaded table: within 1e-6 of
    the oracle's fold then sum."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    rng = np.random.default_rng(700 + n_t)
    accs, gs, folded = [], [], []
    for j in range(n_t):
        n = int(rng.integers(1, 20000))
        a = (rng.standard_normal(n) * 1e-2).astype(np.float32)
        x = (rng.standard_normal(n) * 1e-2).astype(np.float32)
        if j % 2:
            h = oracle.f32_to_bf16_bits(x)
            g = torch.from_numpy(h.view(np.int16).copy()).view(torch.bfloat16).cuda()
        else:
            h = x
            g = torch.from_numpy(x.copy()).cuda()
        f = a.copy()
        oracle.fold_add(f, h)
        accs.append(torch.from_numpy(a).cuda())
        gs.append(g)
        folded.append(f)
    say("fold norm argument table limit", n_t)
    res = torch.zeros(16, dtype=torch.uint8, device="cuda")
    garr, aarr = _lib.tensor_array(gs), _lib.tensor_array(accs)
    ws = torch.empty(L.ely_grad_norm_workspace_bytes(garr, n_t), dtype=torch.uint8, device="cuda")
    _lib.check(L.ely_grad_norm_fold(aarr, garr, n_t, 1.0, res.data_ptr(), ws.data_ptr(), ws.numel(),
                                    _lib.stream_ptr(torch.device("cuda", 0))), "norm fold")
    got = float(res[0:8].view(torch.float64).item())
    want = oracle.sumsq(folded)
    assert abs(got - want) <= 1e-6 * want


@pytest.mark.parametrize("n_t", [48, 49])
def test_argument_table_limit(oracle, n_t):
    """A norm call of up to 48 gradients carries its descriptors in the
    kernel arguments, a longer one uploads a table; either side of the limit
    the sum of squares is within 1e-6 of the oracle's, the one-call clip
    (which reuses the call's descriptors) scales every gradient exactly,
    and a capped grid gives the same bits."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    rng = np.random.default_rng(500 + n_t)
    gs, host = [], []
    for j in range(n_t):
        n = int(rng.integers(1, 20000))
        x = (rng.standard_normal(n) * 1e-2).astype(np.float32)
        if j % 3 == 0:
            h = oracle.f32_to_bf16_bits(x)
            g = torch.from_numpy(h.view(np.int16).copy()).view(torch.bfloat16).cuda()
        else:
            h = x
            g = torch.from_numpy(x.copy()).cuda()
        gs.append(g)
        host.append(h)
    say("norm argument table limit", n_t)
    exact = oracle.sumsq(host)
    s0, norm, coef = _run(L, _lib, gs, 0.5, clip=False)
    assert abs(s0 - exact) <= 1e-6 * exact
    L.ely_set_max_blocks(5)
    try:
        s1, _, _ = _run(L, _lib, gs, 0.5, clip=False)
    finally:
        L.ely_set_max_blocks(0)
    assert np.float64(s1).view(np.uint64) == np.float64(s0).view(np.uint64)
    s2, _, c2 = _run(L, _lib, gs, 0.5, clip=True)
    assert np.float64(s2).view(np.uint64) == np.float64(s0).view(np.uint64) and c2 == coef < 1.0
    for g, h in zip(gs, host):
        if g.dtype == torch.bfloat16:
            assert np.array_equal(bits(g), oracle.f32_to_bf16_bits(oracle.bf16_bits_to_f32(h) * np.float32(coef)))
        else:
            assert np.array_equal(bits(g).view(np.uint32), (h * np.float32(coef)).astype(np.float32).view(np.uint32))
