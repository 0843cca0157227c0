"""Property-based fuzz of the fused AdamW step through the C ABI: ragged
lists of sizes around the kernel's tile, step and quad boundaries (empty
tensors included), each of the five streams of each tensor at its own 0-3
element misalignment, bf16 or fp32 gradients, host or torch op order, weight
decay on or off, a device clip coefficient or none, with or without the bf16
working copy, two steps.  Host order must equal the oracle's HostAdamW
(runtime/optim.py:277-298) bit for bit, parameters, moments and copy; torch
order must stay within 1 ulp of the oracle's foreach-order restatement.
Derandomized, so every run replays the same cases."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from gpu_util import bits, say, ulp_distance

pytestmark = pytest.mark.gpu

FUZZ = settings(max_examples=60, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
SIZES = [0, 1, 3, 4, 5, 1023, 1024, 2047, 2048, 2049, 4095, 4096, 4097, 8191, 12289, 65537]
LR, BETAS, EPS = 1e-2, (0.9, 0.95), 1e-8

tensor_spec = st.tuples(st.sampled_from(SIZES), st.lists(st.sampled_from([0, 0, 1, 2, 3]), min_size=5, max_size=5))


def _view(host: np.ndarray, off: int, dtype) -> torch.Tensor:
    """A device copy of `host` starting `off` elements into its own buffer."""
    buf = torch.zeros(host.size + off, dtype=dtype, device="cuda")
    t = buf[off:]
    src = torch.from_numpy(host.copy())
    t.copy_(src.view(dtype) if dtype == torch.bfloat16 else src)
    return t


@FUZZ
@given(
    specs=st.lists(tensor_spec, min_size=1, max_size=6),
    bf16g=st.booleans(),
    order=st.sampled_from(["host", "torch"]),
    wd=st.sampled_from([0.0, 0.1]),
    clip=st.sampled_from([None, 0.37, 1.0]),
    with_copy=st.booleans(),
    seed=st.integers(0, 2**16),
)
def test_fused_step_matches_the_oracle(oracle, specs, bf16g, order, wd, clip, with_copy, seed):
    from elysium_wan_amd import _lib

    L = _lib.load()
    rng = np.random.default_rng(seed)
    say("adamw fuzz", order, "bf16" if bf16g else "f32", wd, clip, with_copy, [s for s, _ in specs])
    host = []
    dev = []
    for n, offs in specs:
        p = (rng.standard_normal(n) * 0.1).astype(np.float32)
        m = np.zeros(n, np.float32)
        v = np.zeros(n, np.float32)
        c = np.zeros(n, np.uint16)
        host.append([p, m, v, c])
        dev.append([_view(p, offs[0], torch.float32), None, _view(m, offs[2], torch.float32), _view(v, offs[3], torch.float32),
                    _view(c, offs[4], torch.bfloat16) if with_copy else None, offs[1]])
    coef_dev = None if clip is None else torch.tensor([clip], dtype=torch.float32, device="cuda")
    n_t = len(specs)
    ws = torch.empty(L.ely_adamw_workspace_bytes(n_t), dtype=torch.uint8, device="cuda")
    stream = _lib.stream_ptr(torch.device("cuda", 0))
    for step in range(2):
        gs = []
        for (n, _), d in zip(specs, dev):
            g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
            if bf16g:
                g = oracle.f32_to_bf16_bits(g)
            gs.append(g)
            d[1] = _view(g, d[5], torch.bfloat16 if bf16g else torch.float32)
        t = step + 1
        consts = (oracle.host_adamw_consts if order == "host" else oracle.torch_adamw_consts)(LR, BETAS, EPS, wd, t)
        ctab = (_lib.ElyConsts * n_t)()
        for j in range(n_t):
            ctab[j].c[:] = [float(x) for x in np.asarray(consts, dtype=np.float32).reshape(-1)[:8]] + [0.0] * max(0, 8 - len(consts))
        copies = [_lib.ely_tensor(d[4]) if d[4] is not None else _lib.ElyTensor(None, 0, _lib.BF16, 0) for d in dev]
        rc = L.ely_adamw_step(_lib.tensor_array([d[0] for d in dev]), _lib.tensor_array([d[1] for d in dev]),
                              _lib.tensor_array([d[2] for d in dev]), _lib.tensor_array([d[3] for d in dev]),
                              _lib.tensor_array(copies), n_t, ctab, _lib.ORDER_HOST if order == "host" else _lib.ORDER_TORCH,
                              int(wd != 0), None if coef_dev is None else coef_dev.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "adamw fuzz")
        fn = oracle.adamw_host if order == "host" else oracle.adamw_torch
        for (p, m, v, c), g in zip(host, gs):
            fn(p, g, m, v, consts, wd != 0, 1.0 if clip is None else clip, c if with_copy else None)
    torch.cuda.synchronize()
    for (p, m, v, c), d in zip(host, dev):
        for want, got in ((p, d[0]), (m, d[2]), (v, d[3])):
            gb = bits(got)
            if order == "host":
                assert np.array_equal(gb.view(np.uint32), want.view(np.uint32))
            else:
                assert int(ulp_distance(gb.view(np.float32), want).max(initial=0)) <= 1
        if with_copy and order == "host":
            assert np.array_equal(bits(d[4]), c)
