"""Benchmark configs C1, C2 and C3 at their full sizes on one MI355X,
checked through properties that do not need a CPU pass over billions of
elements:

* C1 (the headline: the 2.8B model's stage, 192 tensors, bf16 grads, the
  bf16 working copy, clip, 10 steps): the norm against an fp64 sum of
  squares every step, and one million sampled elements replayed by the
  oracle every step, bit for bit;
* C2 (the 15.8B model's stage: ~7.9B fp32 elements, p/m/v/g resident in
  HBM, 1% of the tensors' gradients x100 so that clipping triggers): the
  global norm against an fp64 sum of squares (within 1e-6), the clip
  coefficient against the oracle's clip_grad_norm_ formula, and a random
  sample of one million elements stepped by the oracle from their gathered
  inputs, bit for bit;
* C3 (the 25.1B model's 4-stage shard: 1,000 vectors of 6,144 interleaved
  with 100 matrices of 6,144 x 10,240, bf16 Student-t gradients): five runs
  from the same seeded inputs give bitwise-identical norms, parameters and
  moments, and a sampled oracle check;
* maximum sizes: one tensor past 2^31 elements through the fused step, and
  an activation past 2^32 codes through the codec (64-bit indexing).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import gpt_block_shapes, say

pytestmark = pytest.mark.gpu

LR, BETAS, EPS, WD, MAX_NORM = 3e-4, (0.9, 0.95), 1e-8, 0.1, 1.0


def _fp64_sumsq(grads) -> float:
    return float(sum(float(g.double().square().sum()) for g in grads))


def test_c2_full_shard_clips_and_steps_exactly(oracle):
    """C2: 25 GPT blocks at d = 5120 (300 tensors, 7,865,984,000 fp32
    elements; p, g, m, v = 126 GB in HBM), fp32 grads N(0, 1e-4) with 3 of
    the 300 tensors (1%) x100."""
    from elysium_wan_amd import optim

    d = 5120
    shapes = [(d,), (d,), (3 * d, d), (3 * d,), (d, d), (d,), (d,), (d,), (4 * d, d), (4 * d,), (d, 4 * d), (d,)] * 25
    gen = torch.Generator(device="cuda").manual_seed(2)
    params, grads = [], []
    hot = {30, 150, 270}
    for i, s in enumerate(shapes):
        params.append(torch.empty(s, device="cuda").normal_(0.0, 0.02, generator=gen).requires_grad_(True))
        grads.append(torch.empty(s, device="cuda").normal_(0.0, 1e-4 * (100.0 if i in hot else 1.0), generator=gen))
    n = sum(p.numel() for p in params)
    assert n == 7_865_984_000
    say("C2 full shard", n)
    opt = optim.FusedAdamW(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order="host", max_norm=MAX_NORM)
    # the inputs of one million sampled elements, saved before the step
    sizes = torch.tensor([p.numel() for p in params], dtype=torch.int64)
    cum = torch.cumsum(sizes, 0)
    flat_idx = torch.randint(0, n, (1_000_000,), generator=torch.Generator().manual_seed(77))
    t_idx = torch.searchsorted(cum, flat_idx, right=True)
    local = flat_idx - (cum[t_idx] - sizes[t_idx])
    saved = {}
    for t in torch.unique(t_idx).tolist():
        sel = local[t_idx == t].cuda()
        saved[t] = (sel, params[t].detach().view(-1)[sel].clone(), grads[t].view(-1)[sel].clone())
    want = _fp64_sumsq(grads)
    opt.step(grads=grads)
    torch.cuda.synchronize()
    norm = float(opt.grad_norm())
    assert abs(norm - want**0.5) <= 1e-6 * want**0.5
    coef = float(opt._norm[12:16].view(torch.float32))
    assert coef < 1.0, "C2's hot tensors make clipping trigger"
    assert coef == oracle.clip_coef(norm, MAX_NORM)
    p_in = np.concatenate([saved[t][1].cpu().numpy() for t in sorted(saved)])
    g_in = np.concatenate([saved[t][2].cpu().numpy() for t in sorted(saved)])
    got_p = np.concatenate([params[t].detach().view(-1)[saved[t][0]].cpu().numpy() for t in sorted(saved)])
    got_m = np.concatenate([opt.state[t]["exp_avg"].view(-1)[saved[t][0]].cpu().numpy() for t in sorted(saved)])
    got_v = np.concatenate([opt.state[t]["exp_avg_sq"].view(-1)[saved[t][0]].cpu().numpy() for t in sorted(saved)])
    m = np.zeros_like(p_in)
    v = np.zeros_like(p_in)
    oracle.adamw_host(p_in, g_in, m, v, np.array(optim.host_consts(LR, BETAS, EPS, WD, 1.0), dtype=np.float32), True, coef)
    assert np.array_equal(got_p.view(np.uint32), p_in.view(np.uint32))
    assert np.array_equal(got_m.view(np.uint32), m.view(np.uint32))
    assert np.array_equal(got_v.view(np.uint32), v.view(np.uint32))
    del opt, params, grads, saved
    torch.cuda.empty_cache()


def test_c1_full_shard_ten_steps_against_the_oracle(oracle):
    """C1, the benchmark's headline shard: 16 GPT blocks at d = 2560 (192
    tensors, 1,258,823,680 fp32 elements), bf16 grads N(0, 1e-4), the bf16
    working copy, weight decay 0.1, clip 1.0, 10 steps.  Every step: the
    norm within 1e-6 of the fp64 sum of squares of all the step's
    gradients, and one million sampled elements (parameter, both moments,
    working copy) equal to the oracle's HostAdamW replaying them from their
    gathered inputs, bit for bit."""
    from elysium_wan_amd import optim

    shapes = gpt_block_shapes(2560) * 16
    gen = torch.Generator(device="cuda").manual_seed(41)
    params = [torch.empty(s, device="cuda").normal_(0.0, 0.02, generator=gen).requires_grad_(True) for s in shapes]
    n = sum(p.numel() for p in params)
    assert n == 1_258_823_680 and len(params) == 192
    opt = optim.FusedAdamW(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order="host", max_norm=MAX_NORM,
                           working_copy=True)
    sizes = torch.tensor([p.numel() for p in params], dtype=torch.int64)
    cum = torch.cumsum(sizes, 0)
    flat_idx = torch.randint(0, n, (1_000_000,), generator=torch.Generator().manual_seed(78))
    t_idx = torch.searchsorted(cum, flat_idx, right=True)
    local = flat_idx - (cum[t_idx] - sizes[t_idx])
    sel = {t: local[t_idx == t].cuda() for t in torch.unique(t_idx).tolist()}
    order = sorted(sel)
    gather = lambda ts: torch.cat([ts[t].detach().reshape(-1)[sel[t]] for t in order])  # noqa: E731
    p = gather(params).cpu().numpy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    cp = np.zeros(p.size, np.uint16)
    ggen = torch.Generator(device="cuda").manual_seed(42)
    for step in range(10):
        grads = [torch.empty(s, device="cuda").normal_(0.0, 1e-4, generator=ggen).to(torch.bfloat16) for s in shapes]
        want = _fp64_sumsq(grads)
        g_in = gather(grads).view(torch.int16).cpu().numpy().view(np.uint16)
        say("C1 full shard, step", step)
        opt.step(grads=grads)
        torch.cuda.synchronize()
        norm = float(opt.grad_norm())
        assert abs(norm - want**0.5) <= 1e-6 * want**0.5, (step, norm, want**0.5)
        coef = float(opt._norm[12:16].view(torch.float32))
        assert coef == oracle.clip_coef(norm, MAX_NORM)
        oracle.adamw_host(p, g_in, m, v, np.array(optim.host_consts(LR, BETAS, EPS, WD, float(step + 1)), dtype=np.float32),
                          True, coef, cp)
        assert np.array_equal(gather(params).cpu().numpy().view(np.uint32), p.view(np.uint32)), step
        assert np.array_equal(gather([opt.state[i]["exp_avg"] for i in range(192)]).cpu().numpy().view(np.uint32), m.view(np.uint32)), step
        assert np.array_equal(gather([opt.state[i]["exp_avg_sq"] for i in range(192)]).cpu().numpy().view(np.uint32), v.view(np.uint32)), step
        assert np.array_equal(gather(opt.working_copies).view(torch.int16).cpu().numpy().view(np.uint16), cp), step
        del grads
    del opt, params
    torch.cuda.empty_cache()


def test_c1_torch_order_equals_torch_adamw_bit_for_bit():
    """C1's shard (192 tensors, 1,258,823,680 elements) under the "adamw"
    recipe (build("adamw"): torch.optim.AdamW's op order) against
    torch.optim.AdamW itself (foreach, the GPU default) on the same GPU,
    fp32 grads N(0, 1e-4), weight decay 0.1, 3 steps: every parameter and
    both moments equal bit for bit (the contract is 1 ulp)."""
    from elysium_wan_amd import optim

    shapes = gpt_block_shapes(2560) * 16
    gen = torch.Generator(device="cuda").manual_seed(43)
    mine = [torch.empty(s, device="cuda").normal_(0.0, 0.02, generator=gen).requires_grad_(True) for s in shapes]
    ref = [p.detach().clone().requires_grad_(True) for p in mine]
    a = optim.build("adamw", mine, LR, weight_decay=WD)
    b = torch.optim.AdamW(ref, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    ggen = torch.Generator(device="cuda").manual_seed(44)
    for step in range(3):
        say("C1 torch order vs torch.optim.AdamW, step", step)
        for p, q in zip(mine, ref):
            g = torch.empty(p.shape, device="cuda").normal_(0.0, 1e-4, generator=ggen)
            p.grad, q.grad = g, g.clone()
        a.step()
        b.step()
        for p, q in zip(mine, ref):
            p.grad = q.grad = None
    torch.cuda.synchronize()
    for i, (p, q) in enumerate(zip(mine, ref)):
        assert torch.equal(p.detach().view(torch.int32), q.detach().view(torch.int32)), i
        assert torch.equal(a.state[p]["exp_avg"].view(torch.int32), b.state[q]["exp_avg"].view(torch.int32)), i
        assert torch.equal(a.state[p]["exp_avg_sq"].view(torch.int32), b.state[q]["exp_avg_sq"].view(torch.int32)), i
    del a, b, mine, ref
    torch.cuda.empty_cache()


def _c3_shard(seed: int):
    """C3: 1,000 vectors of 6,144 interleaved with 100 matrices of
    6,144 x 10,240 (ten vectors, then one matrix), 6,297,600,000 elements;
    params N(0, 0.02) fp32, grads Student-t(df = 3) x 1e-4 in bf16."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    shapes = []
    for _ in range(100):
        shapes += [(6144,)] * 10 + [(6144, 10240)]
    params, grads = [], []
    for s in shapes:
        params.append(torch.empty(s, device="cuda").normal_(0.0, 0.02, generator=gen).requires_grad_(True))
        z = torch.empty(s, device="cuda").normal_(generator=gen)
        c = torch.zeros(s, device="cuda")
        for _ in range(3):
            c.add_(torch.empty(s, device="cuda").normal_(generator=gen).square_())
        grads.append(z.div_(c.div_(3.0).sqrt_()).mul_(1e-4).to(torch.bfloat16))
        del z, c
    return params, grads


def test_c3_ragged_shard_is_bitwise_reproducible(oracle):
    """C3's 1,100-tensor ragged list: five runs of grad-norm + clipped step
    from the same seeded inputs give bit-identical norms and checksums of
    p, m and v; the first run's sampled elements equal the oracle's."""
    from elysium_wan_amd import optim

    sums = []
    for run in range(5):
        params, grads = _c3_shard(33)
        if run == 0:
            n = sum(p.numel() for p in params)
            assert n == 6_297_600_000 and len(params) == 1100
            keep_p = {t: params[t].detach().view(-1)[:4096].clone() for t in range(0, 1100, 37)}
            keep_g = {t: grads[t].view(-1)[:4096].clone() for t in keep_p}
        say("C3 run", run)
        opt = optim.FusedAdamW(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order="host", max_norm=MAX_NORM)
        opt.step(grads=grads)
        torch.cuda.synchronize()
        ck = lambda ts: int(sum(int(t.detach().view(torch.int32).to(torch.int64).sum()) for t in ts))  # noqa: E731
        sums.append((float(opt.grad_norm()), ck(params), ck([opt.state[i]["exp_avg"] for i in range(1100)]), ck([opt.state[i]["exp_avg_sq"] for i in range(1100)])))
        if run == 0:
            coef = float(opt._norm[12:16].view(torch.float32))
            p_in = np.concatenate([keep_p[t].cpu().numpy() for t in keep_p])
            g_in = np.concatenate([keep_g[t].view(torch.int16).cpu().numpy().view(np.uint16) for t in keep_p])
            got = np.concatenate([params[t].detach().view(-1)[:4096].cpu().numpy() for t in keep_p])
            m = np.zeros_like(p_in)
            v = np.zeros_like(p_in)
            oracle.adamw_host(p_in, g_in, m, v, np.array(optim.host_consts(LR, BETAS, EPS, WD, 1.0), dtype=np.float32), True, coef)
            assert np.array_equal(got.view(np.uint32), p_in.view(np.uint32))
        del opt, params, grads
        torch.cuda.empty_cache()
    assert all(s == sums[0] for s in sums), sums


def test_one_tensor_past_two_to_the_31_elements(oracle):
    """Maximum sizes: one fp32 parameter of 2^31 + 4099 elements (bf16 grads,
    clip on) -- 64-bit element and tile indexing.  The norm equals an fp64
    sum within 1e-6; elements at the start, around 2^31 and at the end equal
    the oracle's step of their gathered inputs, bit for bit."""
    from elysium_wan_amd import optim

    n = (1 << 31) + 4099
    gen = torch.Generator(device="cuda").manual_seed(31)
    p = torch.empty(n, device="cuda").normal_(0.0, 0.02, generator=gen).requires_grad_(True)
    g = torch.empty(n, device="cuda").normal_(0.0, 1e-3, generator=gen).to(torch.bfloat16)
    sel = torch.cat([torch.arange(0, 4096), torch.arange((1 << 31) - 4096, (1 << 31) + 4096), torch.arange(n - 4096, n)]).cuda()
    p_in, g_in = p.detach()[sel].clone(), g[sel].clone()
    want = float(g.double().square().sum())
    say("one tensor of", n, "elements")
    opt = optim.FusedAdamW([p], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order="host", max_norm=MAX_NORM, working_copy=True)
    opt.step(grads=[g])
    torch.cuda.synchronize()
    norm = float(opt.grad_norm())
    assert abs(norm - want**0.5) <= 1e-6 * want**0.5
    coef = float(opt._norm[12:16].view(torch.float32))
    pi = p_in.cpu().numpy()
    gi = g_in.view(torch.int16).cpu().numpy().view(np.uint16)
    m, v = np.zeros_like(pi), np.zeros_like(pi)
    cp = np.zeros(pi.size, np.uint16)
    oracle.adamw_host(pi, gi, m, v, np.array(optim.host_consts(LR, BETAS, EPS, WD, 1.0), dtype=np.float32), True, coef, cp)
    assert np.array_equal(p.detach()[sel].cpu().numpy().view(np.uint32), pi.view(np.uint32))
    assert np.array_equal(opt.state[0]["exp_avg"][sel].cpu().numpy().view(np.uint32), m.view(np.uint32))
    assert np.array_equal(opt.state[0]["exp_avg_sq"][sel].cpu().numpy().view(np.uint32), v.view(np.uint32))
    assert np.array_equal(opt.working_copies[0][sel].view(torch.int16).cpu().numpy().view(np.uint16), cp)
    del opt, p, g
    torch.cuda.empty_cache()


def test_fp8_codes_past_two_to_the_32(oracle):
    """Maximum sizes: a [524289, 8192] bf16 activation holds 2^32 + 8192
    codes, so dequantize takes its 64-bit flat indexing; rows before and
    after the 2^32 boundary quantize, dequantize and round-trip like the
    oracle, bit for bit."""
    from elysium_wan_amd import fp8

    rows, cols = (1 << 19) + 1, 8192
    gen = torch.Generator(device="cuda").manual_seed(32)
    x = torch.empty(rows, cols, device="cuda", dtype=torch.bfloat16).normal_(generator=gen)
    say("fp8 rows", rows, "x", cols)
    q, k = fp8.quantize(x, "e4m3")
    d = fp8.dequantize(q, k, torch.bfloat16)
    torch.cuda.synchronize()
    for r in (0, (1 << 19) - 1, 1 << 19):
        xb = x[r : r + 1].view(torch.int16).cpu().numpy().view(np.uint16)
        oq, ok = oracle.quantize(xb, "e4m3")
        assert np.array_equal(q[r : r + 1].view(torch.uint8).cpu().numpy(), oq), r
        assert int(k[r]) == int(ok[0]), r
        assert np.array_equal(d[r : r + 1].view(torch.int16).cpu().numpy().view(np.uint16), oracle.dequantize(oq, ok, "e4m3", "bf16")), r
    del x, q, k, d
    torch.cuda.empty_cache()
