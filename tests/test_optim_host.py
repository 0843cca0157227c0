"""Host-side logic of the optimizer that needs no GPU: the recorded param
group equals torch's own AdamW group (runtime/optim.py:57-69), and an
optimizer is released as soon as its last reference goes, without waiting
for the garbage collector (its parameters and moments are large device
allocations: a reference cycle would hold them past `del opt`)."""

from __future__ import annotations

import gc
import weakref

import pytest
import torch


@pytest.mark.parametrize("recipe", ["adamw", "adamw-host"])
def test_hparams_is_torchs_adamw_group(recipe):
    from elysium_wan_amd import optim

    probe = torch.optim.AdamW([torch.zeros(1, requires_grad=True)], lr=3e-4, **optim.ADAMW)
    want = {k: v for k, v in probe.state_dict()["param_groups"][0].items() if k != "params"}
    if recipe == "adamw-host":
        want["moments"] = "host"
    got = optim.hparams(3e-4, recipe)
    assert got == want and list(got) == list(want)


@pytest.mark.parametrize("order", ["host", "torch"])
def test_optimizer_is_freed_without_the_garbage_collector(order):
    from elysium_wan_amd import optim

    gc.collect()
    gc.disable()
    try:
        opt = optim.FusedAdamW([torch.zeros(3)], lr=1e-3, order=order)  # a frozen tensor: no GPU needed
        ref = weakref.ref(opt)
        assert len(opt.state) == 0
        del opt
        assert ref() is None
    finally:
        gc.enable()


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: asked for more it exits with status 2 and
    says so, before it touches a device."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "8"], capture_output=True, text=True,
                       cwd=root, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and "--gpus 8" in r.stderr
    assert r.stdout == ""
