"""The deterministic global grad-norm on the GPU: within 1e-6 relative of the
oracle's brute-force sum, bitwise identical across runs and grid sizes, and
the clip coefficient and in-place clip of torch's clip_grad_norm_
(TORCH/nn/utils/clip_grad.py:50-183; the reference itself never clips)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import bits, say

pytestmark = pytest.mark.gpu


def _norm(grads, max_norm=1.0):
    from elysium_wan_amd import _lib

    L = _lib.load()
    dev = grads[0].device
    res = torch.zeros(16, dtype=torch.uint8, device=dev)
    arr = _lib.tensor_array(grads)
    ws = _lib.workspace(dev, L.ely_grad_norm_workspace_bytes(arr, len(grads)))
    _lib.check(L.ely_grad_norm(arr, len(grads), float(max_norm), res.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev)), "norm")
    r = res.cpu().numpy()
    return float(r[:8].view(np.float64)[0]), float(r[8:12].view(np.float32)[0]), float(r[12:16].view(np.float32)[0]), r.copy()


def _ragged(seed, n_vec=1000, n_mat=3, d=6144, cols=1024, dtype=torch.bfloat16):
    """Config C3's layout at reduced matrix size: vectors of d interleaved
    with d x cols matrices; Student-t (df 3) x 1e-4 values."""
    gen = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)  # StudentT samples from the global generator
    t = torch.distributions.StudentT(3.0)
    out = []
    per = max(1, n_vec // max(1, n_mat))
    for i in range(n_vec):
        out.append((t.sample((d,)) * 1e-4).to(dtype))
        if i % per == per - 1 and len(out) < n_vec + n_mat:
            out.append((torch.randn(d, cols, generator=gen) * 1e-4).to(dtype))
    return [g.cuda() for g in out]


def test_norm_is_within_1e6_of_the_brute_force_sum(oracle):
    gs = _ragged(1)
    say("norm ragged C3-like", len(gs), sum(g.numel() for g in gs))
    sumsq, norm, coef, _ = _norm(gs, 1.0)
    ref = oracle.sumsq([bits(g) for g in gs])
    assert abs(sumsq - ref) <= 1e-6 * ref
    assert norm == float(np.float32(np.sqrt(sumsq)))
    assert coef == oracle.clip_coef(norm, 1.0)


def test_norm_is_bitwise_reproducible_across_runs_and_grids():
    from elysium_wan_amd import _lib

    gs = _ragged(2) + [torch.randn(1000003, device="cuda") * 1e-3]
    gs.append(torch.randn(77, device="cuda")[1:])  # unaligned fp32 view
    runs = []
    for cap in (0, 0, 0, 0, 0, 1, 13, 999):
        _lib.check(_lib.load().ely_set_max_blocks(cap), "cap")
        try:
            say("norm run, cap", cap)
            runs.append(_norm(gs)[3])
        finally:
            _lib.load().ely_set_max_blocks(0)
    assert all(np.array_equal(runs[0], r) for r in runs[1:])


def test_alignment_does_not_move_a_bit():
    base = torch.randn(200001, device="cuda")
    a = base[:200000].clone()
    b = base[1:].clone()
    b.copy_(a)  # same values, now 16-byte aligned
    buf = torch.empty(200001, device="cuda")
    buf[1:].copy_(a)
    say("norm alignment")
    assert np.array_equal(_norm([a])[3], _norm([buf[1:]])[3])


def test_non_finite_gradients_follow_torch():
    g = torch.ones(100, device="cuda")
    g[3] = float("inf")
    _, norm, coef, _ = _norm([g])
    assert np.isinf(norm) and coef == 0.0
    g[3] = float("nan")
    _, norm, coef, _ = _norm([g])
    assert np.isnan(norm) and np.isnan(coef)


def test_clip_grad_norm_matches_torch(oracle):
    """elysium_wan_amd.optim.clip_grad_norm_ against torch's own on fp32
    grads: the same total norm to 1e-6 and g * coef bit for bit given the
    coefficient (torch sums in fp32, this build in fp64)."""
    from elysium_wan_amd import optim

    gen = torch.Generator().manual_seed(3)
    shapes = [(300, 7), (5000,), (3,)]
    base = [torch.randn(s, generator=gen) * 0.3 for s in shapes]
    ps = [torch.zeros(s, device="cuda", requires_grad=True) for s in shapes]
    qs = [torch.zeros(s, device="cuda", requires_grad=True) for s in shapes]
    for p, q, g in zip(ps, qs, base):
        p.grad = g.cuda()
        q.grad = g.cuda()
    say("clip_grad_norm_ drop-in")
    mine = optim.clip_grad_norm_(ps, 1.0)
    ref = torch.nn.utils.clip_grad_norm_(qs, 1.0)
    assert abs(float(mine) - float(ref)) <= 1e-6 * float(ref)
    coef = oracle.clip_coef(float(mine), 1.0)
    for p, g in zip(ps, base):
        want = (g.numpy() * np.float32(coef)).astype(np.float32)
        assert np.array_equal(bits(p.grad).view(np.uint32), want.view(np.uint32))
    # bf16 gradients are scaled in fp32 and rounded once to bf16
    h = [torch.randn(4097, device="cuda").bfloat16() * 3]
    hp = [torch.zeros(4097, device="cuda", dtype=torch.bfloat16, requires_grad=True)]
    hp[0].grad = h[0].clone()
    total = optim.clip_grad_norm_(hp, 1.0)
    c = oracle.clip_coef(float(total), 1.0)
    want = oracle.f32_to_bf16_bits(oracle.bf16_bits_to_f32(bits(h[0])) * np.float32(c))
    assert np.array_equal(bits(hp[0].grad), want)


def test_clip_grad_norm_in_one_call_scales_every_gradient(oracle):
    """optim.clip_grad_norm_ through ely_grad_norm_clip (the norm, then one
    launch scaling every gradient in place) on a ragged list of bf16 and
    fp32 gradients, unaligned views included, with small-list tiles and, past
    2^29 elements, the large tiles: each gradient equals g * coef rounded once
    to its dtype, with coef the oracle's from the same norm; max_norm 0 zeroes
    the gradients and a negative max_norm flips them, as torch's formula
    does; error_if_nonfinite raises on an Inf before touching anything."""
    from elysium_wan_amd import optim

    gen = torch.Generator(device="cuda").manual_seed(9)

    def grads(big):
        gs = [torch.randn(1_000_003, device="cuda", generator=gen) * 1e-2,
              (torch.randn(4_097, device="cuda", generator=gen) * 3).bfloat16(),
              torch.randn(70_001, device="cuda", generator=gen)[1:],
              (torch.randn(300_001, device="cuda", generator=gen)).bfloat16()[1:]]
        if big:
            gs.append((torch.randn((1 << 29) + 4_099, device="cuda", generator=gen) * 1e-3).bfloat16())
        return gs

    for big, max_norm in ((False, 1.0), (False, 0.0), (False, -2.0), (True, 1.0)):
        gs = grads(big)
        ps = [torch.zeros(g.shape, dtype=g.dtype, device="cuda", requires_grad=True) for g in gs]
        for p, g in zip(ps, gs):
            if g.storage_offset():
                # keep an unaligned view unaligned: a copy one element into a buffer
                buf = torch.empty(g.numel() + 1, dtype=g.dtype, device="cuda")
                buf[1:] = g
                p.grad = buf[1:]
            else:
                p.grad = g.clone()
        say("clip_grad_norm_ one call", "big" if big else "small", max_norm, sum(g.numel() for g in gs))
        total = optim.clip_grad_norm_(ps, max_norm)
        coef = oracle.clip_coef(float(total), max_norm)
        for p, g in zip(ps, gs):
            want = (g.float() * np.float32(coef)).to(g.dtype)
            assert torch.equal(p.grad.view(torch.int16 if g.dtype == torch.bfloat16 else torch.int32),
                               want.view(torch.int16 if g.dtype == torch.bfloat16 else torch.int32))
        if max_norm == 0.0:
            assert coef == 0.0
        del gs, ps
        torch.cuda.empty_cache()
    # error_if_nonfinite: the norm is read first, and an Inf leaves the gradients as they were
    g = torch.randn(10_000, device="cuda")
    g[17] = float("inf")
    p = torch.zeros(10_000, device="cuda", requires_grad=True)
    p.grad = g.clone()
    with pytest.raises(RuntimeError, match="non-finite"):
        optim.clip_grad_norm_([p], 1.0, error_if_nonfinite=True)
    assert torch.equal(p.grad, g)


def test_norm_over_both_load_kinds_is_bitwise_stable_across_grids():
    """A list past the bytes the norm reads last with plain loads (each
    wave's final tiles; the rest nontemporal): both kinds of tiles run, and
    how many of each a wave takes moves with the grid.  The sum of squares
    is bitwise the same for every grid and within 1e-8 of an fp64 sum."""
    from elysium_wan_amd import _lib

    gen = torch.Generator(device="cuda").manual_seed(31)
    gs = [(torch.randn(24 << 20, device="cuda", generator=gen) * 1e-3).bfloat16() for _ in range(10)]
    gs += [torch.randn(5 << 20, device="cuda", generator=gen) * 1e-3 for _ in range(3)]
    gs.append(torch.randn(4097, device="cuda", generator=gen)[1:])  # unaligned tail
    nbytes = sum(g.numel() * g.element_size() for g in gs)
    assert nbytes > (400 << 20)
    exact = sum(float((g.double() ** 2).sum()) for g in gs)
    runs = []
    for cap in (0, 7, 64, 999):
        _lib.check(_lib.load().ely_set_max_blocks(cap), "cap")
        try:
            say("norm over both load kinds, cap", cap, nbytes)
            r = _norm(gs)
            runs.append(r[3])
        finally:
            _lib.load().ely_set_max_blocks(0)
        assert abs(r[0] - exact) <= 1e-8 * exact
    assert all(np.array_equal(runs[0], r) for r in runs[1:])
