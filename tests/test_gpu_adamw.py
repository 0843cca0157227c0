"""The fused clip + AdamW step on the GPU against the oracle, the reference's
golden vectors and torch.optim.AdamW:

* "adamw-host" order: p, m, v and the bf16 working copy bit for bit
  (runtime/optim.py:277-298, pieces.py:192-195), with fp32 and bf16 grads,
  weight decay on and off, clipping on and off, aligned and unaligned
  tensors, any grid size;
* "adamw" order: within 1 ulp of torch.optim.AdamW on the same GPU;
* the torch.optim surface: state_dict layout, resume bit for bit, refusal of
  another recipe, on_param order (the reference's test_host_adamw.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden
from gpu_util import bits, gpt_block_shapes, say, ulp_distance

pytestmark = pytest.mark.gpu

ADAMW = {"betas": (0.9, 0.95), "eps": 1e-8, "weight_decay": 0.0}


def _set_blocks(n: int) -> None:
    from elysium_wan_amd import _lib

    _lib.check(_lib.load().ely_set_max_blocks(n), "ely_set_max_blocks")


@pytest.mark.parametrize("case", ["unit", "decay", "c0"])
def test_reference_golden_steps_bit_for_bit(case):
    """Replays the reference's HostAdamW runs (tests/golden/make_golden.py)
    through optim.build("adamw-host") on the GPU."""
    from elysium_wan_amd import optim

    g = golden("host_adamw.npz")
    lr, b1, b2, eps, wd, steps = g[f"{case}_hyper"]
    numel = [int(n) for n in g[f"{case}_numel"]]
    shapes = [tuple(int(s) for s in row if s) for row in g[f"{case}_shapes"]]
    p0 = torch.from_numpy(g[f"{case}_p0"].copy())
    params = [t.reshape(s).clone().cuda().requires_grad_(True) for t, s in zip(torch.split(p0, numel), shapes)]
    say("golden adamw-host", case)
    opt = optim.build("adamw-host", params, float(lr), betas=(float(b1), float(b2)), eps=float(eps), weight_decay=float(wd))
    for step in range(int(steps)):
        gs = torch.split(torch.from_numpy(g[f"{case}_grads"][step].copy()), numel)
        for p, gr, s in zip(params, gs, shapes):
            p.grad = gr.reshape(s).cuda()
        opt.step()
        opt.zero_grad()
    cat = lambda ts: torch.cat([t.detach().reshape(-1).cpu() for t in ts]).numpy()  # noqa: E731
    assert np.array_equal(cat(params).view(np.uint32), g[f"{case}_p"].view(np.uint32))
    assert np.array_equal(cat([opt.state[i]["exp_avg"] for i in range(len(params))]).view(np.uint32), g[f"{case}_m"].view(np.uint32))
    assert np.array_equal(cat([opt.state[i]["exp_avg_sq"] for i in range(len(params))]).view(np.uint32), g[f"{case}_v"].view(np.uint32))


def _c0_shard(seed: int, gdtype, scale=1e-3, hot=()):
    """Config C0: 3 GPT blocks at d = 768 plus two d-vectors (38 tensors,
    21,265,152 elements); N(0, 0.02) params, N(0, scale) grads; tensors in
    `hot` get grads x100 so the global-norm clip triggers."""
    gen = torch.Generator().manual_seed(seed)
    shapes = gpt_block_shapes(768) * 3 + [(768,), (768,)]
    params = [(torch.randn(s, generator=gen) * 0.02) for s in shapes]
    grads = [(torch.randn(s, generator=gen) * scale * (100.0 if i in hot else 1.0)).to(gdtype) for i, s in enumerate(shapes)]
    return params, grads


def _oracle_steps(oracle, params, grads_per_step, lr, wd, max_norm, copies=True):
    """The oracle's HostAdamW over the flat concatenation, with the clip
    coefficient from the oracle's fp64 norm when max_norm is set."""
    p = np.concatenate([t.reshape(-1).numpy() for t in params]).astype(np.float32)
    m, v = np.zeros_like(p), np.zeros_like(p)
    cp = np.zeros(p.size, dtype=np.uint16) if copies else None
    for step, grads in enumerate(grads_per_step):
        if all(t.dtype == torch.bfloat16 for t in grads):
            gflat = np.concatenate([bits(t).reshape(-1) for t in grads])
        else:  # mixed dtypes: the exact fp32 widening of each part
            gflat = np.concatenate([bits(t.float()).reshape(-1) for t in grads])
        coef = 1.0
        if max_norm is not None:
            norm = float(np.float32(np.sqrt(oracle.sumsq([gflat]))))
            coef = oracle.clip_coef(norm, max_norm)
        c = oracle.host_adamw_consts(lr, (0.9, 0.95), 1e-8, wd, step + 1)
        oracle.adamw_host(p, gflat, m, v, c, wd != 0, coef, cp)
    return p, m, v, cp


@pytest.mark.parametrize("gdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("clip", [None, 1.0])
def test_c0_shard_equals_the_oracle(oracle, gdtype, clip):
    from elysium_wan_amd import optim

    hot = (2, 20) if clip else ()
    params, g0 = _c0_shard(1, gdtype, hot=hot)
    steps = [g0] + [_c0_shard(2 + s, gdtype, hot=hot)[1] for s in range(2)]
    dev = [p.clone().cuda().requires_grad_(True) for p in params]
    say("C0 shard", gdtype, "clip", clip)
    opt = optim.FusedAdamW(dev, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, order="host", max_norm=clip, working_copy=True)
    for gs in steps:
        opt.step(grads=[gr.cuda() for gr in gs])
    if clip:
        assert float(opt.grad_norm()) > clip  # the clip did trigger
    p, m, v, cp = _oracle_steps(oracle, params, steps, 3e-4, 0.1, clip)
    cat = lambda ts: torch.cat([t.detach().reshape(-1) for t in ts]).cpu()  # noqa: E731
    assert np.array_equal(bits(cat(dev)).view(np.uint32), p.view(np.uint32))
    assert np.array_equal(bits(cat([opt.state[i]["exp_avg"] for i in range(len(dev))])).view(np.uint32), m.view(np.uint32))
    assert np.array_equal(bits(cat([opt.state[i]["exp_avg_sq"] for i in range(len(dev))])).view(np.uint32), v.view(np.uint32))
    assert np.array_equal(bits(cat(opt.working_copies)), cp)


def test_unaligned_views_and_grid_sizes_do_not_move_a_bit(oracle):
    """Parameters that are views at odd offsets of one buffer take the element
    path; capping the grid at 1, 7 or 300 blocks changes nothing."""
    from elysium_wan_amd import optim

    gen = torch.Generator().manual_seed(9)
    sizes = [1, 7, 8, 4095, 4097, 100003, 3, 65536]
    flat = torch.randn(sum(sizes) + 1, generator=gen)
    grads = [torch.randn(n, generator=gen) * 1e-2 for n in sizes]
    results = []
    for cap in (0, 1, 7, 300):
        _set_blocks(cap)
        try:
            buf = flat.clone().cuda()
            ps, o = [], 1  # offset 1: every view is 4 bytes off a 16-byte boundary
            for n in sizes:
                ps.append(buf[o : o + n].requires_grad_(True))
                o += n
            say("unaligned views, block cap", cap)
            opt = optim.FusedAdamW(ps, lr=1e-2, betas=(0.9, 0.95), eps=1e-8, order="host", weight_decay=0.1, max_norm=0.5)
            for _ in range(3):
                for p, gr in zip(ps, grads):
                    p.grad = gr.cuda()
                opt.step()
            results.append(bits(buf).copy())
        finally:
            _set_blocks(0)
    assert all(np.array_equal(results[0].view(np.uint32), r.view(np.uint32)) for r in results[1:])
    pf, _, _, _ = _oracle_steps(oracle, [flat[1:]], [[torch.cat(grads)]] * 3, 1e-2, 0.1, 0.5, copies=False)
    assert np.array_equal(results[0][1:].view(np.uint32), pf.view(np.uint32))


_SPECIAL = [0.0, -0.0, 1e-45, -1e-45, 1.1754942e-38, 1e-30, 1e19, -1e19, 1.9e19, 2e19, 1e20, 3.4e38, -3.4e38,
            float("inf"), float("-inf"), float("nan")]


def _nan_as_nan_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """fp32 bits equal, except that any NaN equals any NaN (a NaN made inside
    the arithmetic takes the device's default sign and payload)."""
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_extreme_values_follow_the_oracle(oracle, gdtype):
    """Zeros of both signs, subnormals, gradients whose square overflows fp32
    (v = inf, so sqrt(v) = inf and m / d = 0), +-inf and NaN, in params and
    grads, scattered over a tensor that has both a vector body and an
    element tail: three steps with weight decay equal the oracle, NaN as NaN,
    and the bf16 working copy too."""
    from elysium_wan_amd import optim

    rng = np.random.default_rng(5)
    n = 3 * 4096 + 13
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    pick = rng.choice(n, 200, replace=False)
    p0[pick] = rng.choice(np.array(_SPECIAL, dtype=np.float32), 200)
    gsteps = []
    for _ in range(3):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        pick = rng.choice(n, 400, replace=False)
        g[pick] = rng.choice(np.array(_SPECIAL, dtype=np.float32), 400)
        gsteps.append(torch.from_numpy(g).to(gdtype))
    dev = torch.from_numpy(p0.copy()).cuda().requires_grad_(True)
    say("adamw extreme values", gdtype)
    opt = optim.FusedAdamW([dev], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, order="host", working_copy=True)
    for g in gsteps:
        opt.step(grads=[g.cuda()])
    torch.cuda.synchronize()
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    cp = np.zeros(n, dtype=np.uint16)
    for t, g in enumerate(gsteps):
        oracle.adamw_host(p, bits(g), m, v, oracle.host_adamw_consts(1e-3, (0.9, 0.95), 1e-8, 0.1, t + 1), True, 1.0, cp)
    assert np.isnan(p).any() and np.isinf(v).any() and (np.isinf(p).any() or np.abs(p).max() > 1e38)
    assert _nan_as_nan_equal(bits(dev.detach()), p)
    assert _nan_as_nan_equal(bits(opt.state[0]["exp_avg"]), m)
    assert _nan_as_nan_equal(bits(opt.state[0]["exp_avg_sq"]), v)
    wc = bits(opt.working_copies[0]).astype(np.uint32) << 16
    assert _nan_as_nan_equal(wc.view(np.float32), (cp.astype(np.uint32) << 16).view(np.float32))


@pytest.mark.parametrize("case", ["small", "c0"])
def test_torch_order_is_within_one_ulp_of_torch_adamw(case):
    """optim.build("adamw") against torch.optim.AdamW (foreach, the GPU
    default) on the same GPU, 5 steps, weight decay on, on small ragged
    shapes and on config C0's 38-tensor shard (21,265,152 elements).  The
    contract is 1 ulp; with this image's torch the kernel's fused
    multiply-adds fall where torch's foreach kernels have theirs, so
    parameters, exp_avg and exp_avg_sq come out bit for bit, and the test
    holds it to that."""
    from elysium_wan_amd import optim

    gen = torch.Generator().manual_seed(4)
    if case == "small":
        shapes = [(37, 19), (19,), (5, 3, 7), (1001,), (2560, 64)]
        init = [torch.randn(s, generator=gen) for s in shapes]
    else:
        shapes = gpt_block_shapes(768) * 3 + [(768,), (768,)]
        init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    mine = [t.clone().cuda().requires_grad_(True) for t in init]
    ref = [t.clone().cuda().requires_grad_(True) for t in init]
    a = optim.build("adamw", mine, 1e-2, weight_decay=0.1)
    b = torch.optim.AdamW(ref, lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    say("torch order vs torch.optim.AdamW", case)
    for step in range(5):
        g = torch.Generator(device="cuda").manual_seed(5 + step)
        scale = 10.0 ** (-step % 4) * (1.0 if case == "small" else 1e-3)
        gs = [torch.randn(s, generator=g, device="cuda") * scale for s in shapes]
        for p, q, gr in zip(mine, ref, gs):
            p.grad = gr
            q.grad = gr.clone()
        a.step()
        b.step()
    worst = {}
    for name, xs, ys in (
        ("param", [x.detach() for x in mine], [y.detach() for y in ref]),
        ("exp_avg", [a.state[p]["exp_avg"] for p in mine], [b.state[q]["exp_avg"] for q in ref]),
        ("exp_avg_sq", [a.state[p]["exp_avg_sq"] for p in mine], [b.state[q]["exp_avg_sq"] for q in ref]),
    ):
        d = [ulp_distance(bits(x), bits(y)) for x, y in zip(xs, ys)]
        worst[name] = max(int(x.max()) for x in d)
        exact = sum(int((x == 0).sum()) for x in d) / sum(x.size for x in d)
        say(f"  {name}: max ulp {worst[name]}, bit-identical fraction {exact:.6f}")
    assert max(worst.values()) == 0, worst


def test_state_dict_layout_resume_and_refusals():
    """The reference's test_host_adamw.py contracts on the GPU: torch's AdamW
    layout with "moments": "host", a resume continuing bit for bit, another
    recipe's state refused."""
    from elysium_wan_amd import optim

    def run(params, opt, lo, hi):
        for step in range(lo, hi):
            g = torch.Generator().manual_seed(5 + step)
            for p in params:
                p.grad = (torch.randn(p.shape, generator=g) * 10.0 ** (-step % 4)).cuda()
            opt.step()
            opt.zero_grad()

    gen = torch.Generator().manual_seed(3)
    init = [torch.randn(s, generator=gen) for s in [(37, 19), (19,), (5, 3, 7), (1001,)]]
    full = [t.clone().cuda().requires_grad_(True) for t in init]
    run(full, optim.build("adamw-host", full, 1e-3), 0, 6)
    part = [t.clone().cuda().requires_grad_(True) for t in init]
    opt = optim.build("adamw-host", part, 1e-3)
    run(part, opt, 0, 3)
    sd = opt.state_dict()
    group = dict(sd["param_groups"][0])
    assert group.pop("moments") == "host" and group["params"] == [0, 1, 2, 3]
    for i, p in enumerate(part):
        st = sd["state"][i]
        assert set(st) == {"step", "exp_avg", "exp_avg_sq"} and float(st["step"]) == 3.0
        assert st["exp_avg"].device.type == "cpu" and st["exp_avg"].shape == p.shape
    resumed = [p.detach().clone().requires_grad_(True) for p in part]
    opt2 = optim.build("adamw-host", resumed, 1e-3)
    opt2.load_state_dict(sd)
    run(resumed, opt2, 3, 6)
    assert all(torch.equal(a.view(torch.int32), b.view(torch.int32)) for a, b in zip(full, resumed))
    torch_opt = torch.optim.AdamW([torch.zeros(3, requires_grad=True)], lr=1e-3, **ADAMW)
    with pytest.raises(ValueError, match="another recipe"):
        optim.build("adamw-host", resumed, 1e-3).load_state_dict(torch_opt.state_dict())


def test_on_param_runs_in_parameter_order_and_skips_gradless():
    from elysium_wan_amd import optim

    ps = [torch.zeros(5, device="cuda", requires_grad=True) for _ in range(4)]
    for i in (0, 2, 3):
        ps[i].grad = torch.ones(5, device="cuda")
    seen = []
    optim.build("adamw-host", ps, 1e-3).step(on_param=seen.append)
    assert seen == [0, 2, 3]
    assert torch.equal(ps[1], torch.zeros(5, device="cuda"))


def test_mixed_grad_dtypes_take_one_launch_each(oracle):
    from elysium_wan_amd import optim

    gen = torch.Generator().manual_seed(8)
    init = [torch.randn(1000, generator=gen), torch.randn(77, generator=gen)]
    grads = [torch.randn(1000, generator=gen).bfloat16(), torch.randn(77, generator=gen)]
    ps = [t.clone().cuda().requires_grad_(True) for t in init]
    opt = optim.FusedAdamW(ps, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, order="host", max_norm=1.0)
    opt.step(grads=[g.cuda() for g in grads])
    p, _, _, _ = _oracle_steps(oracle, init, [grads], 1e-3, 0.0, 1.0, copies=False)
    got = torch.cat([x.detach().cpu() for x in ps]).numpy()
    assert np.array_equal(got.view(np.uint32), p.view(np.uint32))


@pytest.mark.parametrize("order", ["host", "torch"])
@pytest.mark.parametrize("gdtype", [torch.bfloat16, torch.float32])
def test_fold_inside_the_update_equals_fold_then_step(order, gdtype):
    """ely_adamw_fold_step / ely_grad_norm_fold: finishing the ordered fold
    (runtime/accumulate.py:93-104) inside the update gives, bit for bit, the
    parameters, moments, working copy and norm of pieces.fold_add followed
    by a plain step; the accumulators are left unwritten."""
    from elysium_wan_amd import optim, pieces

    gen = torch.Generator().manual_seed(21)
    shapes = [(96, 64), (64,), (1000,), (33, 7), (4096,)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    mb = [[(torch.randn(s, generator=gen) * 1e-2).to(gdtype) for s in shapes] for _ in range(3)]
    a_ps = [t.clone().cuda().requires_grad_(True) for t in init]
    b_ps = [t.clone().cuda().requires_grad_(True) for t in init]
    a = optim.FusedAdamW(a_ps, lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, order=order, max_norm=0.5, working_copy=True)
    b = optim.FusedAdamW(b_ps, lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, order=order, max_norm=0.5, working_copy=True)
    say("fold inside the update", order, gdtype)
    for step in range(2):
        parts = [[g.cuda() for g in m] for m in mb]
        accs = [pieces.fold([parts[0][i], parts[1][i]]) for i in range(len(shapes))]
        before = [x.clone() for x in accs]
        a.step(grads=parts[2], acc=accs)
        full = [x.clone() for x in accs]
        for x, g in zip(full, parts[2]):
            pieces.fold_add(x, g)
        b.step(grads=full)
        assert all(torch.equal(x, y) for x, y in zip(accs, before))
    torch.cuda.synchronize()
    assert torch.equal(a.grad_norm().view(torch.int32), b.grad_norm().view(torch.int32))
    for x, y in zip(a_ps, b_ps):
        assert torch.equal(x.detach().view(torch.int32), y.detach().view(torch.int32))
    for i in range(len(shapes)):
        for k in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(a.state[i][k].view(torch.int32), b.state[i][k].view(torch.int32))
        assert torch.equal(a.working_copies[i].view(torch.int16), b.working_copies[i].view(torch.int16))
    # an unaligned view takes the element path and still matches
    big = torch.randn(4097, generator=gen)
    pa, pb = big.clone().cuda()[1:], big.clone().cuda()[1:]
    accv = torch.randn(4097, generator=gen).cuda()[1:]
    gv = torch.randn(4097, generator=gen).cuda()[1:]
    oa = optim.FusedAdamW([pa], lr=1e-3, order=order)
    ob = optim.FusedAdamW([pb], lr=1e-3, order=order)
    oa.step(grads=[gv], acc=[accv])
    ob.step(grads=[accv + gv])
    assert torch.equal(pa.view(torch.int32), pb.view(torch.int32))


def test_step_on_a_side_thread_and_stream():
    """runtime/stage.py:3094-3099 runs step() on a side thread inside
    torch.cuda.stream(side): the launches go to that stream (the main stream
    stays free) and the result equals a step on the main stream."""
    import threading

    from elysium_wan_amd import optim

    gen = torch.Generator().manual_seed(31)
    shapes = [(512, 384), (384,), (70001,)]
    init = [torch.randn(s, generator=gen) for s in shapes]
    grads = [(torch.randn(s, generator=gen) * 1e-2).to(torch.bfloat16).cuda() for s in shapes]
    main = [t.clone().cuda().requires_grad_(True) for t in init]
    side_ps = [t.clone().cuda().requires_grad_(True) for t in init]
    a = optim.FusedAdamW(main, lr=1e-3, betas=(0.9, 0.95), order="host", max_norm=1.0, working_copy=True)
    b = optim.FusedAdamW(side_ps, lr=1e-3, betas=(0.9, 0.95), order="host", max_norm=1.0, working_copy=True)
    side = torch.cuda.Stream()
    seen = []
    errors = []

    def run():
        try:
            with torch.cuda.stream(side):
                for _ in range(3):
                    b.step(grads=grads, on_param=seen.append)
        except Exception as e:  # surfaced below
            errors.append(e)

    say("step on a side thread")
    torch.cuda.synchronize()
    t = threading.Thread(target=run)
    t.start()
    t.join()
    assert not errors, errors
    side.synchronize()
    for _ in range(3):
        a.step(grads=grads)
    torch.cuda.synchronize()
    assert seen == [0, 1, 2] * 3
    for x, y in zip(main, side_ps):
        assert torch.equal(x.detach().view(torch.int32), y.detach().view(torch.int32))
    for x, y in zip(a.working_copies, b.working_copies):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))


def test_two_threads_share_the_upload_ring():
    """Two threads, each on its own stream with its own 60-tensor optimizer
    (past the 48 tensors whose tables ride in the kernel arguments, so every
    norm and update uploads its tables through the library's pinned ring of
    8 slots, which both threads wrap many times): each ends bit for bit where
    the same steps run alone end."""
    import threading

    from elysium_wan_amd import optim

    gen = torch.Generator().manual_seed(37)
    shapes = [(1000 + 37 * i,) for i in range(60)]
    init = [torch.randn(s, generator=gen) for s in shapes]
    grads = [[(torch.randn(s, generator=gen) * 1e-2).to(torch.bfloat16).cuda() for s in shapes] for _ in range(2)]

    def make():
        ps = [t.clone().cuda().requires_grad_(True) for t in init]
        return ps, optim.FusedAdamW(ps, lr=1e-3, betas=(0.9, 0.95), order="host", max_norm=1.0, working_copy=True)

    alone = [make(), make()]
    for j, (_, opt) in enumerate(alone):
        for _ in range(25):
            opt.step(grads=grads[j])
    torch.cuda.synchronize()
    together = [make(), make()]
    errors = []

    def run(j):
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                for _ in range(25):
                    together[j][1].step(grads=grads[j])
                torch.cuda.current_stream().synchronize()
        except Exception as e:  # surfaced below
            errors.append(e)

    say("two threads share the upload ring")
    threads = [threading.Thread(target=run, args=(j,)) for j in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    torch.cuda.synchronize()
    for (pa, oa), (pb, ob) in zip(alone, together):
        for x, y in zip(pa, pb):
            assert torch.equal(x.detach().view(torch.int32), y.detach().view(torch.int32))
        assert torch.equal(oa.grad_norm().view(torch.int32), ob.grad_norm().view(torch.int32))


def test_frozen_parameters_get_no_moments():
    """A frozen tensor (a LoRA base, runtime/optim.py:97-99) is never
    stepped through p.grad and takes no moment memory; one stepped anyway
    through grads= gets moments of its own and the same update."""
    from elysium_wan_amd import optim

    train = torch.randn(1000, device="cuda").requires_grad_(True)
    frozen = torch.randn(1 << 22, device="cuda")  # no requires_grad
    opt = optim.FusedAdamW([train, frozen], lr=1e-3, order="host")
    train.grad = torch.randn(1000, device="cuda")
    opt.step()
    assert opt._flat_m.numel() == 1024 and set(opt.state) == {0}
    g = torch.randn(1 << 22, device="cuda")
    twin = frozen.clone()
    opt.step(grads=[None, g])
    ref = optim.FusedAdamW([twin], lr=1e-3, order="host")
    ref.step(grads=[g])
    assert torch.equal(frozen.view(torch.int32), twin.view(torch.int32))
    assert torch.equal(opt.state[1]["exp_avg_sq"], ref.state[0]["exp_avg_sq"])
