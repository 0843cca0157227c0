"""Property-based fuzz of the fused AdamW step through the C ABI: ragged
lists of sizes around the kernel's tile, step and quad boundaries (empty
tensors included), each of the five streams of each tensor at its own 0-3
element misalignment, bf16 or fp32 gradients, host or torch op order, weight
decay on or off, a device clip coefficient or none, with or without the bf16
working copy, two steps.  Host order must equal the oracle's HostAdamW
(runtime/optim.py:277-298) bit for bit, parameters, moments and copy; torch
order must equal the oracle's foreach-order restatement bit for bit too
(its contract is 1 ulp; kernel and restatement fuse the same operations).
Derandomized, so every run replays the same cases."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from gpu_util import bits, say

pytestmark = pytest.mark.gpu

FUZZ = settings(max_examples=60, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
SIZES = [0, 1, 3, 4, 5, 63, 64, 65, 255, 256, 257, 511, 513, 1023, 1024, 2047, 2048, 2049, 4095, 4096, 4097, 8191, 12289, 65537]
LR, BETAS, EPS = 1e-2, (0.9, 0.95), 1e-8

def _consts_table(oracle, order: str, wd: float, ts):
    """The oracle's constants of each tensor's step t."""
    fn = oracle.host_adamw_consts if order == "host" else oracle.torch_adamw_consts
    return [fn(LR, BETAS, EPS, wd, t) for t in ts]


def _ctab(consts):
    from elysium_wan_amd import _lib

    ctab = (_lib.ElyConsts * len(consts))()
    for j, c in enumerate(consts):
        row = [float(x) for x in np.asarray(c, dtype=np.float32).reshape(-1)[:8]]
        ctab[j].c[:] = row + [0.0] * (8 - len(row))
    return ctab


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
    own_steps=st.booleans(),
    seed=st.integers(0, 2**16),
)
def test_fused_step_matches_the_oracle(oracle, specs, bf16g, order, wd, clip, with_copy, own_steps, seed):
    """own_steps: tensor j at step t + j, so each tensor has its own
    constants and the launch reads them from the uploaded table; otherwise
    the short list's shared constants ride in the kernel arguments."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    rng = np.random.default_rng(seed)
    say("adamw fuzz", order, "bf16" if bf16g else "f32", wd, clip, with_copy, own_steps, [s for s, _ in specs])
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
        consts = _consts_table(oracle, order, wd, [step + 1 + (j if own_steps else 0) for j in range(n_t)])
        ctab = _ctab(consts)
        copies = [_lib.ely_tensor(d[4]) if d[4] is not None else _lib.ElyTensor(None, 0, _lib.BF16, 0) for d in dev]
        rc = L.ely_adamw_step(_lib.tensor_array([d[0] for d in dev]), _lib.tensor_array([d[1] for d in dev]),
                              _lib.tensor_array([d[2] for d in dev]), _lib.tensor_array([d[3] for d in dev]),
                              _lib.tensor_array(copies), n_t, ctab, _lib.ORDER_HOST if order == "host" else _lib.ORDER_TORCH,
                              int(wd != 0), None if coef_dev is None else coef_dev.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "adamw fuzz")
        fn = oracle.adamw_host if order == "host" else oracle.adamw_torch
        for (p, m, v, c), g, cj in zip(host, gs, consts):
            fn(p, g, m, v, cj, wd != 0, 1.0 if clip is None else clip, c if with_copy else None)
    torch.cuda.synchronize()
    for (p, m, v, c), d in zip(host, dev):
        for want, got in ((p, d[0]), (m, d[2]), (v, d[3])):
            gb = bits(got)
            # both orders bit for bit: the torch order's kernel and the
            # oracle's restatement put their fused multiply-adds in the same
            # places (the contract for the torch order is 1 ulp)
            assert np.array_equal(gb.view(np.uint32), want.view(np.uint32)), order
        if with_copy:
            assert np.array_equal(bits(d[4]), c)


fold_spec = st.tuples(st.sampled_from(SIZES), st.lists(st.sampled_from([0, 0, 1, 2, 3]), min_size=6, max_size=6))


@FUZZ
@given(
    specs=st.lists(fold_spec, min_size=1, max_size=6),
    bf16g=st.booleans(),
    order=st.sampled_from(["host", "torch"]),
    wd=st.sampled_from([0.0, 0.1]),
    max_norm=st.sampled_from([None, 0.05, 1e3]),
    with_copy=st.booleans(),
    own_steps=st.booleans(),
    seed=st.integers(0, 2**16),
)
def test_fused_fold_step_matches_the_oracle(oracle, specs, bf16g, order, wd, max_norm, with_copy, own_steps, seed):
    """ely_grad_norm_fold + ely_adamw_fold_step (the last microbatch folded
    inside the norm and the update, runtime/accumulate.py:93-104) against the
    oracle's fold_add followed by its step: the norm within 1e-6 of the
    oracle's fp64 sum of squares of the folded gradients, then both orders
    bit for bit (parameters, moments, working copy), with each of the six
    streams at its own misalignment, over two
    steps, shared or per-tensor constants (own_steps); the accumulators are
    never written."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    rng = np.random.default_rng(seed)
    say("adamw fold fuzz", order, "bf16" if bf16g else "f32", wd, max_norm, with_copy, own_steps, [s for s, _ in specs])
    host, dev = [], []
    for n, offs in specs:
        p = (rng.standard_normal(n) * 0.1).astype(np.float32)
        m, v, c = np.zeros(n, np.float32), np.zeros(n, np.float32), np.zeros(n, np.uint16)
        host.append([p, m, v, c])
        dev.append({"p": _view(p, offs[0], torch.float32), "m": _view(m, offs[2], torch.float32),
                    "v": _view(v, offs[3], torch.float32),
                    "c": _view(c, offs[4], torch.bfloat16) if with_copy else None, "offs": offs})
    n_t = len(specs)
    stream = _lib.stream_ptr(torch.device("cuda", 0))
    res = torch.zeros(16, dtype=torch.uint8, device="cuda")
    for step in range(2):
        gs, accs = [], []
        for (n, _), d in zip(specs, dev):
            a = (rng.standard_normal(n) * 1e-2).astype(np.float32)
            g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
            if bf16g:
                g = oracle.f32_to_bf16_bits(g)
            gs.append(g)
            accs.append(a)
            d["g"] = _view(g, d["offs"][1], torch.bfloat16 if bf16g else torch.float32)
            d["a"] = _view(a, d["offs"][5], torch.float32)
        aarr = _lib.tensor_array([d["a"] for d in dev])
        garr = _lib.tensor_array([d["g"] for d in dev])
        coef_ptr = None
        if max_norm is not None:
            wsn = torch.empty(max(L.ely_grad_norm_workspace_bytes(garr, n_t), 256), dtype=torch.uint8, device="cuda")
            _lib.check(L.ely_grad_norm_fold(aarr, garr, n_t, max_norm, res.data_ptr(), wsn.data_ptr(), wsn.numel(), stream), "norm fold")
            coef_ptr = res.data_ptr() + 12
        consts = _consts_table(oracle, order, wd, [step + 1 + (j if own_steps else 0) for j in range(n_t)])
        ctab = _ctab(consts)
        copies = [_lib.ely_tensor(d["c"]) if d["c"] is not None else _lib.ElyTensor(None, 0, _lib.BF16, 0) for d in dev]
        ws = torch.empty(L.ely_adamw_workspace_bytes(n_t), dtype=torch.uint8, device="cuda")
        rc = L.ely_adamw_fold_step(_lib.tensor_array([d["p"] for d in dev]), aarr, garr,
                                   _lib.tensor_array([d["m"] for d in dev]), _lib.tensor_array([d["v"] for d in dev]),
                                   _lib.tensor_array(copies), n_t, ctab, _lib.ORDER_HOST if order == "host" else _lib.ORDER_TORCH,
                                   int(wd != 0), coef_ptr, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "adamw fold fuzz")
        torch.cuda.synchronize()
        folded = []
        for a, g in zip(accs, gs):
            f = a.copy()
            oracle.fold_add(f, g)
            folded.append(f)
        coef = 1.0
        if max_norm is not None:
            want = oracle.sumsq(folded)
            norm = float(res[8:12].view(torch.float32).item())
            assert abs(float(res[0:8].view(torch.float64).item()) - want) <= 1e-6 * want + 1e-300
            assert abs(norm - want**0.5) <= 1e-6 * want**0.5 + 1e-30
            coef = float(res[12:16].view(torch.float32).item())
            assert coef == oracle.clip_coef(norm, max_norm)
        fn = oracle.adamw_host if order == "host" else oracle.adamw_torch
        for (p, m, v, c), f, cj in zip(host, folded, consts):
            fn(p, f, m, v, cj, wd != 0, coef, c if with_copy else None)
        for a, d in zip(accs, dev):
            assert np.array_equal(bits(d["a"]).view(np.uint32), a.view(np.uint32)), "accumulator written"
    for (p, m, v, c), d in zip(host, dev):
        for want, got in ((p, d["p"]), (m, d["m"]), (v, d["v"])):
            gb = bits(got)
            # both orders bit for bit: the torch order's kernel and the
            # oracle's restatement put their fused multiply-adds in the same
            # places (the contract for the torch order is 1 ulp)
            assert np.array_equal(gb.view(np.uint32), want.view(np.uint32)), order
        if with_copy:
            assert np.array_equal(bits(d["c"]), c)


@pytest.mark.parametrize("n_t", [47, 48, 49, 120])
def test_argument_table_limit(oracle, n_t):
    """Lists of up to 48 tensors at one step carry their descriptors in the
    kernel arguments, longer ones upload a table: either side of the limit
    the step equals the oracle's HostAdamW bit for bit (parameters, moments,
    working copy), ragged sizes, bf16 gradients, clip coefficient."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    rng = np.random.default_rng(1000 + n_t)
    sizes = [int(x) for x in rng.integers(1, 9000, n_t)]
    say("argument table limit", n_t)
    host, dev = [], []
    for n in sizes:
        p = (rng.standard_normal(n) * 0.1).astype(np.float32)
        m, v, c = np.zeros(n, np.float32), np.zeros(n, np.float32), np.zeros(n, np.uint16)
        host.append([p, m, v, c])
        dev.append([_view(p, 0, torch.float32), None, _view(m, 0, torch.float32), _view(v, 0, torch.float32),
                    _view(c, 0, torch.bfloat16)])
    coef_dev = torch.tensor([0.5], dtype=torch.float32, device="cuda")
    ws = torch.empty(L.ely_adamw_workspace_bytes(n_t), dtype=torch.uint8, device="cuda")
    stream = _lib.stream_ptr(torch.device("cuda", 0))
    for step in range(2):
        gs = [oracle.f32_to_bf16_bits((rng.standard_normal(n) * 1e-2).astype(np.float32)) for n in sizes]
        for d, g in zip(dev, gs):
            d[1] = _view(g, 0, torch.bfloat16)
        consts = _consts_table(oracle, "host", 0.1, [step + 1] * n_t)
        rc = L.ely_adamw_step(_lib.tensor_array([d[0] for d in dev]), _lib.tensor_array([d[1] for d in dev]),
                              _lib.tensor_array([d[2] for d in dev]), _lib.tensor_array([d[3] for d in dev]),
                              _lib.tensor_array([d[4] for d in dev]), n_t, _ctab(consts), _lib.ORDER_HOST, 1,
                              coef_dev.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "argument table limit")
        for (p, m, v, c), g, cj in zip(host, gs, consts):
            oracle.adamw_host(p, g, m, v, cj, True, 0.5, c)
    torch.cuda.synchronize()
    for (p, m, v, c), d in zip(host, dev):
        for want, got in ((p, d[0]), (m, d[2]), (v, d[3])):
            assert np.array_equal(bits(got).view(np.uint32), want.view(np.uint32))
        assert np.array_equal(bits(d[4]), c)
