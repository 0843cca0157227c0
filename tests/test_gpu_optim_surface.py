"""The torch.optim surface of the fused optimizer on the GPU, as the
reference's callers use it:

* the "adamw" recipe's state keyed by parameter tensor, read and assigned
  the way runtime/stage.py:2265-2271 (pieces checkpoint) and :2642-2646
  (pieces resume) do, resuming bit for bit;
* a state entry replaced, a load_state_dict and a frozen parameter stepped
  through grads= all reach the kernel (the descriptor cache follows the
  moments' pointers), checked against the oracle;
* torch.optim.AdamW's load_state_dict semantics for the "adamw" recipe
  (hyperparameters adopted, a torch AdamW's own state loaded, amsgrad
  refused) and its lr read from the param group at every step;
* on_param: the update issued in parameter-ordered groups, each group's
  parameters released right after it, with the bits of the single launch,
  for HBM and host moments (runtime/optim.py:164-170,
  runtime/stage.py:3080-3099)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import bits, gpt_block_shapes, say, ulp_distance

pytestmark = pytest.mark.gpu


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().view(torch.int32)


def test_pieces_state_is_keyed_by_master_and_resumes_bit_for_bit():
    """pieces.adamw's state is read per master tensor for the checkpoint
    (stage.py:2265-2271) and assigned per master tensor on resume
    (stage.py:2642-2646); three more steps after the resume equal an
    uninterrupted run bit for bit."""
    from elysium_wan_amd import pieces

    gen = torch.Generator().manual_seed(51)
    shapes = [(96, 80), (80,), (1001,), (17, 33)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    grads = [[(torch.randn(s, generator=gen) * 1e-2) for s in shapes] for _ in range(6)]

    def run(opt, masters, lo, hi):
        for step in range(lo, hi):
            pieces.step_unit(opt, masters, [g.cuda() for g in grads[step]])

    full = [t.clone().cuda().requires_grad_(True) for t in init]
    run(pieces.adamw(full, 1e-3), full, 0, 6)
    masters = [t.clone().cuda().requires_grad_(True) for t in init]
    popt = pieces.adamw(masters, 1e-3)
    say("pieces checkpoint and resume")
    run(popt, masters, 0, 3)
    st = popt.state
    keys = list(st)
    assert len(keys) == len(masters) and all(a is b for a, b in zip(keys, masters))
    assert all(m in st for m in masters)
    assert all(st[m] is st[i] for i, m in enumerate(masters))
    saved = {
        i: {
            "master": m.detach().cpu().clone(),
            "exp_avg": st[m]["exp_avg"].cpu().clone(),
            "exp_avg_sq": st[m]["exp_avg_sq"].cpu().clone(),
            "step": st[m]["step"].clone(),
        }
        for i, m in enumerate(masters)
    }
    assert all(float(s["step"]) == 3.0 for s in saved.values())
    resumed = [saved[i]["master"].cuda().requires_grad_(True) for i in range(len(masters))]
    popt2 = pieces.adamw(resumed, 1e-3)
    with torch.no_grad():
        for i, m in enumerate(resumed):
            popt2.state[m] = {
                "step": saved[i]["step"],
                "exp_avg": saved[i]["exp_avg"].to(m.device),
                "exp_avg_sq": saved[i]["exp_avg_sq"].to(m.device),
            }
    assert all(float(popt2.state[m]["step"]) == 3.0 for m in resumed)
    run(popt2, resumed, 3, 6)
    assert all(torch.equal(_i32(a), _i32(b)) for a, b in zip(full, resumed))
    with pytest.raises(KeyError):
        popt2.state[torch.zeros(3, device="cuda")]


def test_replaced_state_load_and_frozen_step_reach_the_kernel(oracle):
    """A moment tensor replaced in a state entry, a load_state_dict, and a
    frozen tensor stepped through grads= (moments of its own) each reach the
    next launch: every step equals the oracle's HostAdamW, bit for bit."""
    from elysium_wan_amd import optim

    rng = np.random.default_rng(7)
    p0 = (rng.standard_normal(5000) * 0.1).astype(np.float32)
    f0 = (rng.standard_normal(3000) * 0.1).astype(np.float32)
    train = torch.from_numpy(p0.copy()).cuda().requires_grad_(True)
    frozen = torch.from_numpy(f0.copy()).cuda()
    opt = optim.FusedAdamW([train, frozen], lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, order="host")
    host = [[p0.copy(), np.zeros_like(p0), np.zeros_like(p0)], [f0.copy(), np.zeros_like(f0), np.zeros_like(f0)]]
    steps = [0, 0]

    def step_both(label):
        gs = [(rng.standard_normal(5000) * 1e-2).astype(np.float32), (rng.standard_normal(3000) * 1e-2).astype(np.float32)]
        say("surface:", label)
        opt.step(grads=[torch.from_numpy(g).cuda() for g in gs])
        for k, g in enumerate(gs):
            steps[k] += 1
            p, m, v = host[k]
            oracle.adamw_host(p, g, m, v, oracle.host_adamw_consts(1e-2, (0.9, 0.95), 1e-8, 0.1, steps[k]), True)
        torch.cuda.synchronize()
        for k, t in enumerate((train, frozen)):
            p, m, v = host[k]
            assert np.array_equal(bits(t).view(np.uint32), p.view(np.uint32)), label
            assert np.array_equal(bits(opt.state[k]["exp_avg"]).view(np.uint32), m.view(np.uint32)), label
            assert np.array_equal(bits(opt.state[k]["exp_avg_sq"]).view(np.uint32), v.view(np.uint32)), label

    step_both("first step")
    step_both("cached tables")
    # a state entry's moment replaced by another tensor
    new_m = (rng.standard_normal(5000) * 1e-3).astype(np.float32)
    opt.state[0]["exp_avg"] = torch.from_numpy(new_m.copy()).cuda()
    host[0][1] = new_m.copy()
    step_both("replaced exp_avg")
    # a checkpoint round trip: the frozen tensor's moments are made anew
    sd = opt.state_dict()
    sd = {"state": {i: {k: (v.clone() if torch.is_tensor(v) else v) for k, v in s.items()} for i, s in sd["state"].items()},
          "param_groups": sd["param_groups"]}
    opt.load_state_dict(sd)
    step_both("after load_state_dict")
    # a state entry dropped starts again from zero moments at step 0
    del opt.state[1]
    host[1][1][:] = 0
    host[1][2][:] = 0
    steps[1] = 0
    step_both("after del state[1]")


def test_torch_recipe_loads_state_with_torch_semantics():
    """build("adamw") follows torch.optim.AdamW.load_state_dict: a torch
    AdamW's own state_dict loads and both continue within 1 ulp; the saved
    lr is adopted; amsgrad and a different parameter count are refused."""
    from elysium_wan_amd import optim

    gen = torch.Generator().manual_seed(61)
    shapes = [(64, 48), (48,), (5000,)]
    init = [torch.randn(s, generator=gen) for s in shapes]
    grads = [[torch.randn(s, generator=gen) * 1e-2 for s in shapes] for _ in range(5)]
    ref = [t.clone().cuda().requires_grad_(True) for t in init]
    topt = torch.optim.AdamW(ref, lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)

    def tstep(opt, ps, step):
        for p, g in zip(ps, grads[step]):
            p.grad = g.cuda()
        opt.step()

    for step in range(3):
        tstep(topt, ref, step)
    mine = [p.detach().clone().requires_grad_(True) for p in ref]
    sd = topt.state_dict()
    sd["param_groups"][0]["lr"] = 5e-3  # a scheduler's lr, saved with the state
    for g in topt.param_groups:
        g["lr"] = 5e-3
    fopt = optim.build("adamw", mine, 1e-2, weight_decay=0.1)
    say("torch recipe: load torch's own AdamW state")
    fopt.load_state_dict(sd)
    assert fopt.param_groups[0]["lr"] == 5e-3 and fopt.lr == 5e-3
    assert all(float(fopt.state[p]["step"]) == 3.0 for p in mine)
    for step in (3, 4):
        tstep(topt, ref, step)
        tstep(fopt, mine, step)
    worst = max(int(ulp_distance(bits(a.detach()), bits(b.detach())).max()) for a, b in zip(mine, ref))
    assert worst == 0, worst  # the contract is 1 ulp; this image's torch is matched bit for bit
    # a scheduler changing the group's lr between steps takes effect, as in torch
    for opt in (topt, fopt):
        opt.param_groups[0]["lr"] = 2e-3
    tstep(topt, ref, 0)
    tstep(fopt, mine, 0)
    worst = max(int(ulp_distance(bits(a.detach()), bits(b.detach())).max()) for a, b in zip(mine, ref))
    assert worst == 0, worst  # the contract is 1 ulp; this image's torch is matched bit for bit
    bad = topt.state_dict()
    bad["param_groups"][0]["amsgrad"] = True
    with pytest.raises(ValueError, match="amsgrad"):
        optim.build("adamw", [p.detach().clone().requires_grad_(True) for p in ref], 1e-2).load_state_dict(bad)
    with pytest.raises(ValueError, match="doesn't match the size"):
        optim.build("adamw", [p.detach().clone().requires_grad_(True) for p in ref[:2]], 1e-2).load_state_dict(topt.state_dict())


@pytest.mark.parametrize("recipe", ["adamw-host-hbm", "adamw-host", "adamw"])
def test_on_param_releases_groups_in_order_with_the_single_launch_bits(recipe):
    """step(on_param=...) issues the update in parameter-ordered groups of
    release_elems elements and calls on_param(i) right after the group
    holding i: the order is the parameter order (gradless parameters
    skipped), each callback sees its own group issued before the next group
    is, and parameters, moments and working copies equal the single launch's
    bit for bit (mixed bf16/fp32 gradients, clip on)."""
    from elysium_wan_amd import optim

    gen = torch.Generator().manual_seed(71)
    shapes = gpt_block_shapes(256) * 3
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    kw = dict(lr=1e-3, max_norm=0.5, working_copy=True, weight_decay=0.1)
    if recipe == "adamw-host-hbm":
        kw["moments"] = "device"
    name = "adamw" if recipe == "adamw" else "adamw-host"
    a_ps = [t.clone().cuda().requires_grad_(True) for t in init]
    b_ps = [t.clone().cuda().requires_grad_(True) for t in init]
    a = optim.build(name, a_ps, **kw)
    b = optim.build(name, b_ps, release_elems=200_000, **kw)
    seen = []
    issue = b._issue

    def traced_issue(grp, idx, *rest):
        seen.append(("issued", [idx[j] for j in grp]))
        issue(grp, idx, *rest)

    b._issue = traced_issue

    def release(i):
        seen.append(i)

    say("on_param groups", recipe)
    for step in range(3):
        gs = [(torch.randn(s, generator=gen) * 1e-2) for s in shapes]
        gs = [g.bfloat16() if k % 3 else g for k, g in enumerate(gs)]
        gs[5] = None  # a parameter without a gradient this step
        a.step(grads=[None if g is None else g.cuda() for g in gs])
        b.step(grads=[None if g is None else g.cuda() for g in gs], on_param=release)
    torch.cuda.synchronize()
    # every group is issued, then exactly its parameters are released, in order
    released, k, groups = [], 0, 0
    while k < len(seen):
        tag, members = seen[k]
        assert tag == "issued"
        assert seen[k + 1 : k + 1 + len(members)] == members
        released += members
        k += 1 + len(members)
        groups += 1
    assert released == [i for i in range(len(shapes)) if i != 5] * 3
    assert groups > 9, "the test must cut each step into several groups"
    for x, y in zip(a_ps, b_ps):
        assert torch.equal(_i32(x), _i32(y))
    assert 5 not in a.state and 5 not in b.state  # never stepped: no state, as torch
    for i in range(len(shapes)):
        if i == 5:
            continue
        for k in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(_i32(a.state[i][k].cuda()), _i32(b.state[i][k].cuda())), (i, k)
        assert torch.equal(a.working_copies[i].view(torch.int16), b.working_copies[i].view(torch.int16))
