"""The "adamw-host" recipe with its moments in pinned host memory, streamed
through the GPU in chunks (runtime/optim.py:176-204, 301-363): the
reference's own contracts (tests/unit/test_host_adamw.py) on the GPU --
chunking, staging slots and the copy pipeline move no bit, so the streamed
step equals the HBM-resident step; the moments live in host memory and
checkpoint in torch's layout; promote moves them to the GPU without changing
a bit; the planner prices the recipe at 8 device bytes per element."""

from __future__ import annotations

import pytest
import torch

from gpu_util import gpt_block_shapes, say

pytestmark = pytest.mark.gpu


def _params(seed=3, shapes=((37, 19), (19,), (5, 3, 7), (1001,))):
    """tests/unit/test_host_adamw.py:20-23 (moved to the GPU)."""
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=g).cuda().requires_grad_(True) for s in shapes]


def _grads(params, step, seed=5, dtype=torch.float32):
    """tests/unit/test_host_adamw.py:26-28."""
    g = torch.Generator().manual_seed(seed + step)
    return [(torch.randn(p.shape, generator=g) * 10.0 ** (-step % 4)).to(dtype).cuda() for p in params]


def _train(make, params, steps=4, dtype=torch.float32, fold=False):
    opt = make(params)
    for step in range(steps):
        gs = _grads(params, step, dtype=dtype)
        if fold:
            accs = [(torch.randn(p.shape, generator=torch.Generator().manual_seed(90 + step)) * 1e-2).cuda() for p in params]
            opt.step(grads=gs, acc=accs)
        else:
            opt.step(grads=gs)
    torch.cuda.synchronize()
    return opt


def _same(a, b) -> bool:
    for i, (x, y) in enumerate(zip(a.params, b.params)):
        if not torch.equal(x.detach().view(torch.int32), y.detach().view(torch.int32)):
            return False
        for k in ("exp_avg", "exp_avg_sq"):
            if not torch.equal(a.state[i][k].cpu().view(torch.int32), b.state[i][k].cpu().view(torch.int32)):
                return False
        if a.working_copies is not None and not torch.equal(a.working_copies[i].view(torch.int16), b.working_copies[i].view(torch.int16)):
            return False
    return True


@pytest.mark.parametrize("chunk,slots,pipeline", [(7, 2, True), (7, 3, False), (64, 3, None), (1 << 24, 3, None)])
def test_streamed_moments_equal_resident_moments(chunk, slots, pipeline):
    """test_host_adamw.py:50-55, 154-167: updated in place through the GPU's
    mapping of the pinned buffers (the default), or chunk k in slot k %
    slots, refilled across parameter boundaries, staged or serial -- the
    parameters and moments equal the HBM-resident run's, bit for bit."""
    from elysium_wan_amd import optim

    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, order="host", max_norm=1.0, working_copy=True)
    say("host moments", chunk, slots, pipeline)
    dev = _train(lambda ps: optim.FusedAdamW(ps, **hp), _params())
    host = _train(lambda ps: optim.FusedAdamW(ps, moments="host", chunk=chunk, slots=slots, pipeline=pipeline, **hp), _params())
    assert all(host.state[i]["exp_avg"].device.type == "cpu" for i in host.state)
    assert (host._mapped is not None) == (pipeline is None)
    assert _same(dev, host)


@pytest.mark.parametrize("pipeline", [None, True])
@pytest.mark.parametrize("order", ["host", "torch"])
def test_streamed_c0_shard_with_bf16_grads_and_fold(order, pipeline):
    """Config C0's layout (3 GPT blocks at d = 768, 21.3M elements), in place
    or in chunks of 2^20 through 3 slots, bf16 gradients folded into fp32
    accumulators inside the update: equal to the resident run."""
    from elysium_wan_amd import optim

    shapes = tuple(gpt_block_shapes(768) * 3 + [(768,), (768,)])
    hp = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, order=order, max_norm=1.0, working_copy=True)
    say("host moments C0", order, pipeline)
    dev = _train(lambda ps: optim.FusedAdamW(ps, **hp), _params(7, shapes), steps=2, dtype=torch.bfloat16, fold=True)
    host = _train(lambda ps: optim.FusedAdamW(ps, moments="host", chunk=1 << 20, pipeline=pipeline, **hp), _params(7, shapes), steps=2,
                  dtype=torch.bfloat16, fold=True)
    assert _same(dev, host)


def test_recipe_lives_in_host_memory_checkpoints_and_promotes():
    """test_host_adamw.py:80-96, 170-185: build("adamw-host") keeps its
    moments in host memory, checkpoints host tensors in torch's layout, and
    promote() moves them to the GPU without moving a bit."""
    from elysium_wan_amd import optim

    assert optim.state_bytes_per_param("adamw-host") == 8 and optim.state_bytes_per_param("adamw") == 16
    ref = _train(lambda ps: optim.build("adamw-host", ps, 1e-3, moments="device"), _params(), steps=6)
    params = _params()
    opt = optim.build("adamw-host", params, 1e-3)
    for step in range(3):
        opt.step(grads=_grads(params, step))
    sd = opt.state_dict()
    assert sd["param_groups"][0]["moments"] == "host"
    assert all(sd["state"][i]["exp_avg"].device.type == "cpu" for i in range(4))
    moved = opt.promote(8 * (37 * 19 + 19))
    assert moved == 8 * (37 * 19 + 19) and opt.resident == {0, 1}
    assert opt.state[0]["exp_avg"].device.type == "cuda" and opt.state[2]["exp_avg"].device.type == "cpu"
    for step in range(3, 6):
        opt.step(grads=_grads(params, step))
    torch.cuda.synchronize()
    assert _same(ref, opt)
    sd = opt.state_dict()
    assert all(sd["state"][i]["exp_avg"].device.type == "cpu" for i in range(4))
    # a resumed host-moment optimizer continues bit for bit
    params2 = [p.detach().clone().requires_grad_(True) for p in params]
    opt2 = optim.build("adamw-host", params2, 1e-3)
    opt2.load_state_dict(sd)
    ref.step(grads=_grads(params, 6))
    opt2.step(grads=_grads(params2, 6))
    torch.cuda.synchronize()
    assert all(torch.equal(a.detach().view(torch.int32), b.detach().view(torch.int32)) for a, b in zip(ref.params, params2))


def test_a_swapped_host_moment_is_refused_before_any_launch():
    """Host moments are views of the optimizer's pinned buffers, which the
    update reaches in place; a state tensor replaced by another host tensor
    is refused with ValueError before anything is launched, and the
    parameters stay as they were."""
    from elysium_wan_amd import optim

    params = _params()
    opt = optim.build("adamw-host", params, 1e-3)
    opt.step(grads=_grads(params, 0))
    torch.cuda.synchronize()
    before = [p.detach().clone() for p in params]
    opt.state[2]["exp_avg"] = torch.zeros_like(opt.state[2]["exp_avg"])
    say("swapped host moment")
    with pytest.raises(ValueError, match="pinned moment buffer"):
        opt.step(grads=_grads(params, 1))
    torch.cuda.synchronize()
    assert all(torch.equal(a, b.detach()) for a, b in zip(before, params))
    assert all(float(opt.state[i]["step"]) == 1.0 for i in range(len(params)))


def _check_set(n: int, seed: int):
    """benchmarks/wan/check_host_adamw.py:19-22: four tensors of n // 4,
    n // 4, n // 2 - 7 and 7 elements, N(0, 1) (CPU generator, seeded)."""
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=g) for s in (n // 4, n // 4, n // 2 - 7, 7)]


@pytest.mark.parametrize("arm", ["in_place", "staged", "serial", "staged_half_resident", "in_place_half_resident"])
def test_check_host_adamw_bits_equal_the_cpu(oracle, arm):
    """benchmarks/wan/check_host_adamw.py:25-55 on this build: "adamw-host"
    over 3,000,001 elements in four tensors, lr 3e-4 and runtime/spec.py's
    AdamW, three steps of grads N(0, 1) x 10^-(step % 5) (seed 100 + step),
    half the moments promoted to the GPU after the first step in the
    half-resident arms -- parameters and moments equal the CPU's HostAdamW
    arithmetic (the oracle) bit for bit, for every arm of the reference's
    check plus the in-place default."""
    import numpy as np

    from elysium_wan_amd import optim

    n = 3_000_001
    init = _check_set(n, 1)
    params = [t.clone().cuda().requires_grad_(True) for t in init]
    pipeline = {"in_place": None, "staged": True, "serial": False,
                "staged_half_resident": True, "in_place_half_resident": None}[arm]
    opt = optim.build("adamw-host", params, 3e-4, pipeline=pipeline)
    p = np.concatenate([t.numpy() for t in init])
    m, v = np.zeros_like(p), np.zeros_like(p)
    say("check_host_adamw arm", arm)
    for step in range(3):
        if step == 1 and arm.endswith("half_resident"):
            moved = opt.promote(int(0.5 * 8 * n))
            assert 0 < moved <= 4 * n and opt.resident
        g = torch.Generator().manual_seed(100 + step)
        gs = [torch.randn(t.shape, generator=g) * 10.0 ** (-(step % 5)) for t in init]
        for x, gr in zip(params, gs):
            x.grad = gr.cuda()
        opt.step()
        opt.zero_grad()
        oracle.adamw_host(p, np.concatenate([gr.numpy() for gr in gs]), m, v,
                          oracle.host_adamw_consts(3e-4, (0.9, 0.95), 1e-8, 0.0, step + 1), False)
    got = np.concatenate([x.detach().cpu().numpy() for x in params])
    assert np.array_equal(got.view(np.uint32), p.view(np.uint32))
    gm = np.concatenate([opt.state[i]["exp_avg"].cpu().numpy().reshape(-1) for i in range(4)])
    gv = np.concatenate([opt.state[i]["exp_avg_sq"].cpu().numpy().reshape(-1) for i in range(4)])
    assert np.array_equal(gm.view(np.uint32), m.view(np.uint32))
    assert np.array_equal(gv.view(np.uint32), v.view(np.uint32))
