"""The ordered microbatch fold (accumulate.OrderedAccumulator, the drop-in
for runtime/accumulate.py:15-137) on the GPU, feeding the fused update:
parts handed in out of order and through quarantine fold in microbatch
order, bit for bit against the oracle's left fold; with defer_last the last
microbatch is folded inside the update (FusedAdamW.step(grads, acc)) and
the step equals the oracle's fold-then-HostAdamW bit for bit, norm and clip
included (runtime/stage.py:3002-3024 then runtime/optim.py:145-174)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from gpu_util import bits, say

pytestmark = pytest.mark.gpu

SHAPES = [(96, 64), (64,), (4097,), (33, 7), (8192,)]


def _parts(seed: int, m: int, dtype):
    gen = torch.Generator().manual_seed(seed)
    return [[(torch.randn(s, generator=gen) * 1e-2).to(dtype) for s in SHAPES] for _ in range(m)]


def _oracle_fold(oracle, parts, i):
    """Microbatch order, tensor i: the first part widened, then fold_add."""
    acc = bits(parts[0][i].float()).reshape(-1).copy()
    for mb in range(1, len(parts)):
        oracle.fold_add(acc, bits(parts[mb][i]).reshape(-1))
    return acc


@pytest.mark.parametrize("gdtype", [torch.bfloat16, torch.float32])
def test_out_of_order_parts_fold_in_order_and_into_the_update(oracle, gdtype):
    from elysium_wan_amd import accumulate, optim

    M = 4
    parts = _parts(3, M, gdtype)
    gen = torch.Generator().manual_seed(4)
    init = [torch.randn(s, generator=gen) * 0.02 for s in SHAPES]
    ps = [t.clone().cuda().requires_grad_(True) for t in init]
    opt = optim.FusedAdamW(ps, lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, order="host", max_norm=0.5,
                           working_copy=True)
    plain = accumulate.OrderedAccumulator(range(M))
    deferred = accumulate.OrderedAccumulator(range(M), defer_last=True)
    # arrivals: mb 2 before mb 1, mb 3 (the last) early, mb 1 quarantined then released;
    # tensors of one microbatch in scrambled order (fold_part, RUNTIME-I21)
    arrivals = [(0, [4, 0, 2, 1, 3]), (2, [1, 3, 0, 4, 2]), (3, [0, 1, 2, 3, 4]), (1, [3, 2, 4, 0, 1])]
    say("ordered fold", gdtype)
    for acc in (plain, deferred):
        for mb, order in arrivals:
            if mb == 1:
                acc.add(mb, [parts[mb][i].cuda() for i in range(len(SHAPES))], verified=False)
                assert not acc.complete() and acc.pos == 1
                acc.release(mb)
            else:
                for i in order:
                    acc.fold_part(mb, i, len(SHAPES), parts[mb][i].cuda(), torch.float32)
                acc.end_part(mb)
        assert acc.complete()
    grads, accs = deferred.step_inputs()
    assert all(g.dtype == gdtype for g in grads) and all(a.dtype == torch.float32 for a in accs)
    for i in range(len(SHAPES)):
        prefix = bits(parts[0][i].float()).reshape(-1).copy()
        for mb in (1, 2):
            oracle.fold_add(prefix, bits(parts[mb][i]).reshape(-1))
        assert np.array_equal(bits(accs[i]).reshape(-1).view(np.uint32), prefix.view(np.uint32)), i
    opt.step(grads=grads, acc=accs)
    torch.cuda.synchronize()
    full = [_oracle_fold(oracle, parts, i) for i in range(len(SHAPES))]
    for i, s in enumerate(plain.result()):
        assert np.array_equal(bits(s).reshape(-1).view(np.uint32), full[i].view(np.uint32)), i
    for i, s in enumerate(deferred.result()):
        assert np.array_equal(bits(s).reshape(-1).view(np.uint32), full[i].view(np.uint32)), i
    g = np.concatenate(full)
    norm = float(np.float32(np.sqrt(oracle.sumsq([g]))))
    assert abs(float(opt.grad_norm()) - norm) <= 1e-6 * norm
    coef = float(opt._norm[12:16].view(torch.float32))
    assert coef == oracle.clip_coef(float(opt.grad_norm()), 0.5)
    p = np.concatenate([t.reshape(-1).numpy() for t in init])
    m, v, cp = np.zeros_like(p), np.zeros_like(p), np.zeros(p.size, np.uint16)
    oracle.adamw_host(p, g, m, v, oracle.host_adamw_consts(1e-2, (0.9, 0.95), 1e-8, 0.1, 1), True, coef, cp)
    got = np.concatenate([bits(t).reshape(-1) for t in ps])
    assert np.array_equal(got.view(np.uint32), p.view(np.uint32))
    assert np.array_equal(np.concatenate([bits(opt.state[i]["exp_avg"]).reshape(-1) for i in range(len(SHAPES))]).view(np.uint32),
                          m.view(np.uint32))
    assert np.array_equal(np.concatenate([bits(c).reshape(-1) for c in opt.working_copies]), cp)


def test_one_microbatch_defers_its_only_part(oracle):
    """With a single microbatch the held part is the whole gradient: no
    accumulator, and the step widens it in registers exactly as the
    reference's widening copy would."""
    from elysium_wan_amd import accumulate, optim

    parts = _parts(5, 1, torch.bfloat16)
    acc = accumulate.OrderedAccumulator([0], defer_last=True)
    acc.add(0, [t.cuda() for t in parts[0]])
    grads, accs = acc.step_inputs()
    assert accs is None and all(g.dtype == torch.bfloat16 for g in grads)
    gen = torch.Generator().manual_seed(6)
    init = [torch.randn(s, generator=gen) * 0.02 for s in SHAPES]
    a = [t.clone().cuda().requires_grad_(True) for t in init]
    b = [t.clone().cuda().requires_grad_(True) for t in init]
    oa = optim.FusedAdamW(a, lr=1e-2, order="host")
    ob = optim.FusedAdamW(b, lr=1e-2, order="host")
    oa.step(grads=grads, acc=accs)
    full = acc.result()
    assert all(s.dtype == torch.bfloat16 for s in full)  # no widening dtype was named: the reference's clone
    ob.step(grads=[t.float() for t in full])
    torch.cuda.synchronize()
    assert all(torch.equal(x.detach().view(torch.int32), y.detach().view(torch.int32)) for x, y in zip(a, b))


@settings(max_examples=25, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
@given(
    m=st.integers(1, 5),
    bf16=st.booleans(),
    defer=st.booleans(),
    quarantine=st.integers(-1, 4),
    perm_seed=st.integers(0, 2**16),
)
def test_ordered_fold_fuzz_equals_the_oracle(oracle, m, bf16, defer, quarantine, perm_seed):
    """Random microbatch counts, part dtypes, arrival orders of every
    (microbatch, tensor) part and an optional quarantined microbatch:
    result() equals the oracle's left fold in microbatch order bit for bit,
    and with defer_last the prefix sums and held parts are the oracle's
    prefix fold and last microbatch."""
    import random

    from elysium_wan_amd import accumulate

    dtype = torch.bfloat16 if bf16 else torch.float32
    parts = _parts(100 + perm_seed % 97, m, dtype)
    acc = accumulate.OrderedAccumulator(range(m), defer_last=defer)
    q = quarantine if 0 <= quarantine < m else None
    events = [(mb, i) for mb in range(m) for i in range(len(SHAPES))]
    random.Random(perm_seed).shuffle(events)
    say("ordered fold fuzz", m, dtype, defer, q)
    if q is not None:
        acc.add(q, [parts[q][i].cuda() for i in range(len(SHAPES))], verified=False)
    seen = {mb: 0 for mb in range(m)}
    for mb, i in events:
        if mb == q:
            continue
        acc.fold_part(mb, i, len(SHAPES), parts[mb][i].cuda(), torch.float32)
        seen[mb] += 1
        if seen[mb] == len(SHAPES):
            acc.end_part(mb)
    if q is not None:
        assert not acc.complete()
        acc.release(q)
    assert acc.complete()
    if defer:
        grads, accs = acc.step_inputs()
        for i in range(len(SHAPES)):
            assert torch.equal(grads[i].cpu(), parts[m - 1][i])
            if m > 1:
                assert np.array_equal(bits(accs[i]).reshape(-1).view(np.uint32),
                                      _oracle_fold(oracle, parts[: m - 1], i).view(np.uint32))
        assert accs is None or m > 1
    for i, s in enumerate(acc.result()):
        assert np.array_equal(bits(s.float()).reshape(-1).view(np.uint32), _oracle_fold(oracle, parts, i).view(np.uint32))


@settings(max_examples=30, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
@given(
    n=st.sampled_from([1, 3, 4, 5, 1023, 1024, 4097, 100_003]),
    bf16g=st.booleans(),
    acc_off=st.integers(0, 3),
    g_off=st.integers(0, 3),
    seed=st.integers(0, 2**16),
)
def test_fold_into_a_bf16_sum_equals_the_oracle_and_torch(oracle, n, bf16g, acc_off, g_off, seed):
    """ely_fold_add_bf16 (the ordered fold into a bf16 sum,
    runtime/accumulate.py:101-102): bit for bit the oracle's fold and torch's
    own add_ on the GPU, with the sum and the part at their own element
    offsets (vector and scalar paths), NaN/Inf/-0 sprinkled in."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    rng = np.random.default_rng(seed)
    acc = oracle.f32_to_bf16_bits((rng.standard_normal(n) * 10.0 ** rng.integers(-3, 3)).astype(np.float32))
    x = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    x[rng.random(n) < 0.01] = np.inf
    x[rng.random(n) < 0.01] = np.nan
    x[rng.random(n) < 0.01] = -0.0
    g = oracle.f32_to_bf16_bits(x) if bf16g else x
    say("bf16-sum fold", n, bf16g, acc_off, g_off)
    abuf = torch.zeros(n + acc_off, dtype=torch.bfloat16, device="cuda")
    a = abuf[acc_off:]
    a.copy_(torch.from_numpy(acc.view(np.int16).copy()).view(torch.bfloat16))
    gdt = torch.bfloat16 if bf16g else torch.float32
    gbuf = torch.zeros(n + g_off, dtype=gdt, device="cuda")
    gt = gbuf[g_off:]
    gt.copy_(torch.from_numpy(g.view(np.int16).copy()).view(torch.bfloat16) if bf16g else torch.from_numpy(g.copy()))
    ref = a.clone()
    ref.add_(gt)  # torch's own add on the GPU
    _lib.check(L.ely_fold_add_bf16(a.data_ptr(), gt.data_ptr(), _lib.dtype_code(gt), n, _lib.stream_ptr(a.device)), "fold bf16")
    want = acc.copy()
    oracle.fold_add_bf16(want, g)
    got = bits(a)
    assert np.array_equal(got, want)
    assert np.array_equal(got, bits(ref))


def test_ordered_fold_of_bf16_parts_keeps_a_bf16_sum(oracle):
    """bf16 parts folded with no wider dtype asked for (fold_part without
    `dtype`, or add): the sum stays bf16, first part copied, then each later
    part added in fp32 and rounded to bf16, as the reference's add_ on a bf16
    tensor; out-of-order arrival changes no bit."""
    from elysium_wan_amd import accumulate

    M = 4
    parts = _parts(77, M, torch.bfloat16)
    acc = accumulate.OrderedAccumulator(range(M))
    say("bf16-sum ordered fold")
    for mb in (2, 0, 3, 1):
        for i in reversed(range(len(SHAPES))):
            acc.fold_part(mb, i, len(SHAPES), parts[mb][i].cuda())
        acc.end_part(mb)
    assert acc.complete()
    for i, s in enumerate(acc.result()):
        assert s.dtype == torch.bfloat16
        want = bits(parts[0][i]).reshape(-1).copy()
        for mb in range(1, M):
            oracle.fold_add_bf16(want, bits(parts[mb][i]).reshape(-1))
        assert np.array_equal(bits(s).reshape(-1), want), i
