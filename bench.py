"""Benchmark of the per-stage update path on one MI355X (benchmark config C1:
one of the 2 pipeline stages of the 2.8B model).

    python bench.py [--steps K] [--warmup W] [--gpus 1]

A step is one optimizer step of the stage's shard with every input resident
in HBM: 16 GPT blocks at d = 2560 (192 tensors, 1,258,823,680 fp32 params),
bf16 grads N(0, 1e-4), fp32 m and v, a bf16 working copy out, AdamW lr 3e-4,
betas 0.9/0.95, eps 1e-8, weight decay 0.1, global-norm clip 1.0 -- i.e.
the deterministic grad-norm launch plus the fused clip + AdamW launch.
`value` is params/s of the whole timed step.  The fp8 boundary codec is
timed beside it on C1's activation [8, 2048, 2560] (e4m3) and gradient
(e5m2), per-row scaling, rotating through enough copies that no launch
reads from the 256 MB MALL, and swept over config C4 ([16, 4096, 8192]
Student-t activation and N(0, 1e-5) gradient; e4m3 and e5m2; per-row and
per-tensor) with relative error and digests of the exact bytes and scales.

Prints one JSON line (rank 0):
  roofline      -- the fused AdamW kernel: algorithmic bytes per launch
                   (28 B/elem: read p, g(bf16), m, v; write p, m, v, copy)
                   over its average duration from HIP events on its stream;
  cpu_baseline  -- the reference's own CPU path for the step (torch's
                   clip_grad_norm_ + AdamW(foreach=False) + the bf16 cast)
                   on every core torch is given on this host, over a
                   bounded prefix of the same shard; the 1-thread figure and
                   the oracle's C port sit in extra.cpu_context.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
D_MODEL, N_BLOCKS = 2560, 16
LR, BETAS, EPS, WD, MAX_NORM = 3e-4, (0.9, 0.95), 1e-8, 0.1, 1.0
ADAM_BYTES_PER_ELEM = 28  # bf16 grads, bf16 copy out
NORM_BYTES_PER_ELEM = 2
CODEC_BYTES_PER_ELEM = 3  # bf16 in / fp8 out (quantize); fp8 in / bf16 out (dequantize)
ROUNDTRIP_BYTES_PER_ELEM = 4  # bf16 in, bf16 out (fp8.roundtrip, nothing else written)
C1_CODEC_COPIES, C1_CODEC_ITERS = 8, 20  # C1 codec leg: rotating inputs, launches per timed group
C4_CODEC_ITERS = 10  # C4 codec leg: launches per timed group
CAL_ELEMS = 1 << 28  # calibration cast of the --pmc passes


_T0 = time.perf_counter()


def log(*a):
    print(f"[{time.perf_counter() - _T0:6.1f}s]", *a, file=sys.stderr, flush=True)


def block_shapes(d: int):
    return [(d,), (d,), (3 * d, d), (3 * d,), (d, d), (d,), (d,), (d,), (4 * d, d), (4 * d,), (d, 4 * d), (d,)]


def make_shard(device):
    """C1's shard: params N(0, 0.02) fp32, grads N(0, 1e-4) bf16, generated on
    the device (seeded)."""
    gen = torch.Generator(device=device).manual_seed(1234)
    shapes = block_shapes(D_MODEL) * N_BLOCKS
    params, grads = [], []
    for s in shapes:
        p = torch.empty(s, dtype=torch.float32, device=device)
        p.normal_(0.0, 0.02, generator=gen)
        g = torch.empty(s, dtype=torch.float32, device=device)
        g.normal_(0.0, 1e-4, generator=gen)
        params.append(p.requires_grad_(True))
        grads.append(g.to(torch.bfloat16))
        del g
    return params, grads


def time_events(fn, iters, stream):
    """Average duration (ms) of fn() over iters launches, HIP events on
    `stream`, after one untimed call (code-object load, first-touch)."""
    fn(0)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        starts[i].record(stream)
        fn(i)
        ends[i].record(stream)
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / iters


def time_back_to_back(fn, iters, stream):
    """Average period (ms) of iters back-to-back launches of fn() between one
    pair of HIP events on `stream`, after one untimed call: the launches
    queue behind each other, so their dispatch latency overlaps the previous
    launch's tail."""
    fn(0)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(iters):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def bench_optimizer(args, device, stream):
    params, grads = make_shard(device)
    log(f"C1 shard: {len(params)} tensors, {sum(p.numel() for p in params)} elements")
    return measure_shard(params, grads, device, stream, args.steps, args.warmup)


def measure_shard(params, grads, device, stream, steps, warmup, order="host"):
    """Times optimizer steps of one shard (grad-norm launch + fused clip +
    AdamW launch, bf16 working copy out) by wall clock around `steps` whole
    steps, then each of the two launches alone with HIP events on the
    launch stream."""
    from elysium_wan_amd import _lib, optim

    n_elem = sum(p.numel() for p in params)
    opt = optim.FusedAdamW(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order=order, max_norm=MAX_NORM, working_copy=True)
    for _ in range(warmup):
        opt.step(grads=grads)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        opt.step(grads=grads)
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / steps

    # Per-kernel durations: the same two launches through the C ABI, with HIP
    # events on the launch stream between them.
    L = _lib.load()
    sptr = _lib.stream_ptr(device)
    garr = _lib.tensor_array(grads)
    nws = _lib.workspace(device, L.ely_grad_norm_workspace_bytes(garr, len(grads)))
    res = torch.zeros(16, dtype=torch.uint8, device=device)
    n = len(params)
    parr = _lib.tensor_array(params)
    marr = _lib.tensor_array([opt.state[i]["exp_avg"] for i in range(n)])
    varr = _lib.tensor_array([opt.state[i]["exp_avg_sq"] for i in range(n)])
    carr = _lib.tensor_array(opt.working_copies)
    consts = (_lib.ElyConsts * n)()
    base_step = float(opt.state[0]["step"])
    aws = torch.empty(L.ely_adamw_workspace_bytes(n), dtype=torch.uint8, device=device)

    def norm(_):
        _lib.check(L.ely_grad_norm(garr, n, MAX_NORM, res.data_ptr(), nws.data_ptr(), nws.numel(), sptr), "norm")

    iters = max(steps, 5)
    cfn = optim.host_consts if order == "host" else optim.torch_consts
    per_step = [cfn(LR, BETAS, EPS, WD, base_step + 1 + i) for i in range(iters)]
    code = _lib.ORDER_HOST if order == "host" else _lib.ORDER_TORCH

    def adam(i):
        for j in range(n):
            consts[j].c[:] = per_step[i]
        _lib.check(L.ely_adamw_step(parr, garr, marr, varr, carr, n, consts, code, 1, res.data_ptr() + 12, aws.data_ptr(), aws.numel(), sptr), "adamw")

    norm_ms = time_events(norm, iters, stream)
    adam_ms = time_events(adam, iters, stream)
    out = {
        "n_elem": n_elem,
        "step_s": step_s,
        "norm_ms": norm_ms,
        "adam_ms": adam_ms,
        "grad_norm": float(opt.grad_norm()),
        "clip_coef": float(opt._norm[12:16].view(torch.float32)),
    }
    del opt
    return out


def _shard_rates(o, grad_bytes, tensors):
    """Rates of one measure_shard result: AdamW reads p, g, m, v and writes
    p, m, v and the bf16 copy (26 + grad_bytes B/elem); the norm reads g."""
    n = o["n_elem"]
    adam_gbs = n * (26 + grad_bytes) / o["adam_ms"] / 1e6
    return {
        "tensors": tensors,
        "n_elem": n,
        "step_ms": o["step_s"] * 1e3,
        "params_per_s": n / o["step_s"],
        "adamw_ms": o["adam_ms"],
        "adamw_GBs": adam_gbs,
        "adamw_frac": adam_gbs / HBM_PEAK_GBS,
        "grad_norm_ms": o["norm_ms"],
        "grad_norm_GBs": n * grad_bytes / o["norm_ms"] / 1e6,
        "clip_coef": o["clip_coef"],
    }


def config_shard(name, device):
    """The other optimizer configs at their full sizes, generated on the
    device (seeded):
    C0 -- 3 GPT blocks at d = 768 + 2 vectors (38 tensors, 21,265,152
          elements), fp32 grads N(0, 1e-3);
    C2 -- 25 GPT blocks at d = 5120 (300 tensors, 7,865,984,000 elements),
          fp32 grads N(0, 1e-4) with 3 tensors (1%) x100 so the clip triggers;
    C3 -- 1,000 vectors of 6,144 interleaved with 100 matrices of
          6,144 x 10,240 (1,100 tensors, 6,297,600,000 elements), bf16 grads
          Student-t (df = 3) x 1e-4.
    Params are N(0, 0.02) fp32 throughout."""
    gen = torch.Generator(device=device).manual_seed({"c0": 10, "c2": 12, "c3": 13}[name])
    if name == "c0":
        shapes, gdt, scale, hot = block_shapes(768) * 3 + [(768,), (768,)], torch.float32, 1e-3, set()
    elif name == "c2":
        shapes, gdt, scale, hot = block_shapes(5120) * 25, torch.float32, 1e-4, {30, 150, 270}
    else:
        shapes, gdt, scale, hot = [], torch.bfloat16, 1e-4, set()
        for _ in range(100):
            shapes += [(6144,)] * 10 + [(6144, 10240)]
    params, grads = [], []
    for i, sh in enumerate(shapes):
        params.append(torch.empty(sh, device=device).normal_(0.0, 0.02, generator=gen).requires_grad_(True))
        if name == "c3":
            z = torch.empty(sh, device=device).normal_(generator=gen)
            c = torch.zeros(sh, device=device)
            for _ in range(3):
                c.add_(torch.empty(sh, device=device).normal_(generator=gen).square_())
            grads.append(z.div_(c.div_(3.0).sqrt_()).mul_(scale).to(gdt))
            del z, c
        else:
            g = torch.empty(sh, device=device).normal_(0.0, scale * (100.0 if i in hot else 1.0), generator=gen)
            grads.append(g if gdt == torch.float32 else g.to(gdt))
    return params, grads


def bench_configs(device, stream, names=("c0", "c2", "c3"), steps=3, warmup=1):
    """The fused step over configs C0, C2 and C3 at their full sizes: the
    same launches as the headline C1 measurement, on a small
    launch-bound shard (C0), a 126 GB resident shard whose clip triggers
    (C2) and a 1,100-tensor ragged shard (C3)."""
    out = {}
    for name in names:
        params, grads = config_shard(name, device)
        log(f"{name} shard: {len(params)} tensors, {sum(p.numel() for p in params)} elements")
        gbytes = grads[0].element_size()
        # C0's steps take ~0.2 ms: time 50 of them, so the window's start and
        # sync do not weigh on the figure; the large shards take `steps`
        k, w = (max(steps, 50), max(warmup, 5)) if name == "c0" else (steps, warmup)
        o = measure_shard(params, grads, device, stream, k, w)
        out[name] = _shard_rates(o, gbytes, len(params))
        del params, grads
        torch.cuda.empty_cache()
    return out


def bench_torch_order(device, stream, steps=5, warmup=2):
    """C1's step with the "adamw" recipe (build("adamw"): torch.optim.AdamW's
    op order, TORCH/optim/adam.py:688-800) instead of "adamw-host"'s: the
    same bytes, other arithmetic."""
    params, grads = make_shard(device)
    o = measure_shard(params, grads, device, stream, steps, warmup, order="torch")
    del params, grads
    return _shard_rates(o, 2, 192)


def bench_placement(device, stream, hold_gib=150):
    """C1's step with its shard allocated while `hold_gib` GiB of other device
    memory are held, so that its pages come from another physical range
    than a fresh process's first allocation. The kernel and the bytes are
    the same; what changes is the DRAM side (how long the L2 channels wait
    for DRAM credits)."""
    hold = torch.empty(hold_gib << 30, dtype=torch.uint8, device=device)
    params, grads = make_shard(device)
    o = measure_shard(params, grads, device, stream, 3, 1)
    del params, grads, hold
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    r = _shard_rates(o, 2, 192)
    r["held_GiB"] = hold_gib
    return r


def _activations(device, rows, cols, copies, seed):
    """bf16 N(0, 1) with 0.1% of the elements x50 (config C1's activation recipe)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    xs = []
    for _ in range(copies):
        x = torch.empty(rows, cols, device=device)
        x.normal_(generator=gen)
        mask = torch.rand(rows, cols, device=device, generator=gen) < 1e-3
        xs.append(torch.where(mask, x * 50.0, x).to(torch.bfloat16))
        del x, mask
    return xs


def _c4_inputs(device, seed):
    """Config C4's two inputs of shape [16, 4096, 8192] bf16: the activation,
    Student-t (df = 3) with 0.01% of the elements set to +-1e4, and the
    gradient, N(0, 1e-5)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    shape = (16 * 4096, 8192)
    z = torch.empty(shape, device=device).normal_(generator=gen)
    c = torch.zeros(shape, device=device)
    for _ in range(3):
        c.add_(torch.empty(shape, device=device).normal_(generator=gen).square_())
    z.div_(c.div_(3.0).sqrt_())
    del c
    n = z.numel()
    idx = torch.randint(0, n, (n // 10000,), generator=gen, device=device)
    sign = torch.randint(0, 2, idx.shape, generator=gen, device=device).float() * 2 - 1
    z.view(-1)[idx] = 1e4 * sign
    act = z.to(torch.bfloat16)
    del z
    grad = torch.empty(shape, device=device).normal_(0.0, 1e-5, generator=gen).to(torch.bfloat16)
    return {"activation": act, "gradient": grad}


def bench_codec(device, stream, rows, cols, copies, iters=20, per_tensor=False, xs=None, fmts=("e4m3", "e5m2"), stats=False,
                back_to_back=False):
    """Quantize, dequantize and the fused round trip (bf16 <-> fp8, per-row
    or per-tensor) of a [rows, cols] activation, rotating through `copies` inputs so that
    launches stream from HBM rather than the 256 MB MALL. With `stats`, the
    round trip of the first input is also reported, outside the timed
    region: relative L2 error of dequantize(quantize(x)) against x, the
    range of the exponents k, and SHA-256 digests of the fp8 bytes and k.
    With `back_to_back`, each leg is also timed as one queue of launches."""
    import hashlib

    from elysium_wan_amd import _lib

    L = _lib.load()
    sptr = _lib.stream_ptr(device)
    n = rows * cols
    xs = xs if xs is not None else _activations(device, rows, cols, copies, 7)
    copies = len(xs)
    qs = [torch.empty(rows, cols, dtype=torch.uint8, device=device) for _ in range(copies)]
    qr, qc = (1, n) if per_tensor else (rows, cols)
    ks = [torch.empty(qr, dtype=torch.int32, device=device) for _ in range(copies)]
    outs = [torch.empty(rows, cols, dtype=torch.bfloat16, device=device) for _ in range(copies)]
    ws = _lib.workspace(device, L.ely_fp8_workspace_bytes(qr, qc, _lib.BF16))
    out = {}
    for fmt in fmts:
        f = _lib.FMT[fmt]

        def quant(i, f=f):
            j = i % copies
            _lib.check(L.ely_fp8_quantize(xs[j].data_ptr(), _lib.BF16, qr, qc, f, qs[j].data_ptr(), ks[j].data_ptr(), ws.data_ptr(), ws.numel(), sptr), "q")

        def deq(i, f=f):
            j = i % copies
            _lib.check(L.ely_fp8_dequantize(qs[j].data_ptr(), ks[j].data_ptr(), qr, qc, f, outs[j].data_ptr(), _lib.BF16, sptr), "dq")

        def rt(i, f=f):
            # fp8.roundtrip (model/fp8.py:56-63): quantize and dequantize fused, bf16 in and out
            j = i % copies
            _lib.check(L.ely_fp8_roundtrip(xs[j].data_ptr(), _lib.BF16, qr, qc, f, outs[j].data_ptr(), None, None, ws.data_ptr(), ws.numel(), sptr), "rt")

        for i in range(copies):
            quant(i)
        q_ms = time_events(quant, iters, stream)
        d_ms = time_events(deq, iters, stream)
        r_ms = time_events(rt, iters, stream)
        out[fmt] = {
            "quantize_ms": q_ms,
            "quantize_GBs": n * CODEC_BYTES_PER_ELEM / q_ms / 1e6,
            "dequantize_ms": d_ms,
            "dequantize_GBs": n * CODEC_BYTES_PER_ELEM / d_ms / 1e6,
            "roundtrip_ms": r_ms,
            "roundtrip_GBs": n * ROUNDTRIP_BYTES_PER_ELEM / r_ms / 1e6,
        }
        if per_tensor:
            # the one-pass form given the exponent (fp8.quantize(...,
            # per_tensor=True, k_hint=k)): a right hint (x read once) and a
            # wrong one (the fixup pass at the true exponent), and the round
            # trip with a right hint; the codes equal the split path's
            hws = _lib.workspace(device, L.ely_fp8_hint_workspace_bytes(n))
            hit = torch.zeros(1, dtype=torch.int32, device=device)
            k_true = [int(kk.item()) for kk in ks]
            qh = [torch.empty_like(qq) for qq in qs]

            def qhint(i, f=f, off=0):
                j = i % copies
                _lib.check(L.ely_fp8_quantize_hint(xs[j].data_ptr(), _lib.BF16, n, f, k_true[j] + off, None, qh[j].data_ptr(),
                                                   ks[j].data_ptr(), None, hit.data_ptr(), hws.data_ptr(), hws.numel(), sptr), "qh")

            def rthint(i, f=f):
                j = i % copies
                _lib.check(L.ely_fp8_quantize_hint(xs[j].data_ptr(), _lib.BF16, n, f, k_true[j], None, None, ks[j].data_ptr(),
                                                   outs[j].data_ptr(), hit.data_ptr(), hws.data_ptr(), hws.numel(), sptr), "rth")

            h_ms = time_events(qhint, iters, stream)
            hit_after = int(hit.item())
            m_ms = time_events(lambda i: qhint(i, off=1), iters, stream)
            miss_after = int(hit.item())
            rh_ms = time_events(rthint, iters, stream)
            qhint(0)
            torch.cuda.synchronize()
            out[fmt]["hint"] = {
                "quantize_hit_ms": h_ms,
                "quantize_hit_GBs": n * CODEC_BYTES_PER_ELEM / h_ms / 1e6,
                "quantize_miss_ms": m_ms,
                "quantize_miss_GBs": n * CODEC_BYTES_PER_ELEM / m_ms / 1e6,
                "roundtrip_hit_ms": rh_ms,
                "roundtrip_hit_GBs": n * ROUNDTRIP_BYTES_PER_ELEM / rh_ms / 1e6,
                "hit_flags": [hit_after, miss_after],
                "codes_equal_split_path": bool(torch.equal(qh[0], qs[0])),
            }
            del qh
        if back_to_back:
            # the same launches queued back to back (one event pair around all)
            out[fmt]["back_to_back_GBs"] = {
                "quantize": n * CODEC_BYTES_PER_ELEM / time_back_to_back(quant, iters, stream) / 1e6,
                "dequantize": n * CODEC_BYTES_PER_ELEM / time_back_to_back(deq, iters, stream) / 1e6,
                "roundtrip": n * ROUNDTRIP_BYTES_PER_ELEM / time_back_to_back(rt, iters, stream) / 1e6,
            }
        if stats:
            quant(0)
            deq(0)
            torch.cuda.synchronize()
            x64 = xs[0].double()
            err = float((outs[0].double() - x64).norm() / x64.norm())
            del x64
            out[fmt].update({
                "rel_l2_error": err,
                "k_min": int(ks[0].min()),
                "k_max": int(ks[0].max()),
                "fp8_sha256": hashlib.sha256(qs[0].cpu().numpy().tobytes()).hexdigest(),
                "k_sha256": hashlib.sha256(ks[0].cpu().numpy().tobytes()).hexdigest(),
            })
    del xs, qs, outs
    return out


def bench_c4(device, stream, iters=C4_CODEC_ITERS):
    """Config C4's sweep: {activation, gradient} x {e4m3, e5m2} x {per-row
    (8,192 wide), per-tensor}, encode -> decode, with timings, relative
    error, exponent range and digests of the exact fp8 bytes and scales."""
    inputs = _c4_inputs(device, 44)
    rows, cols = inputs["activation"].shape
    out = {}
    for name, x in inputs.items():
        out[name] = {}
        for per_tensor in (False, True):
            out[name]["per_tensor" if per_tensor else "per_row"] = bench_codec(device, stream, rows, cols, 2, iters=iters, per_tensor=per_tensor, xs=[x, x.clone()], stats=True)
            torch.cuda.empty_cache()
    del inputs
    return out


def bench_fold(device, stream, iters=5):
    """The ordered fold finished inside the update (ely_adamw_fold_step:
    read acc 4 + g 2, p m v 12; write p m v 12 + copy 2 = 32 B/elem) against
    the fold pass (ely_fold_add, 10 B/elem) followed by the plain step on the
    fp32 sum (30 B/elem), over C1's shard with bf16 last-microbatch grads."""
    from elysium_wan_amd import _lib, optim

    params, grads = make_shard(device)
    n = len(params)
    n_elem = sum(p.numel() for p in params)
    accs = [torch.empty_like(p).normal_(0.0, 1e-4) for p in params]
    opt = optim.FusedAdamW(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order="host", working_copy=True)
    opt.step(grads=grads, acc=accs)  # allocates the moments
    torch.cuda.synchronize()
    L = _lib.load()
    sptr = _lib.stream_ptr(device)
    parr, garr, aarr = _lib.tensor_array(params), _lib.tensor_array(grads), _lib.tensor_array(accs)
    marr = _lib.tensor_array([opt.state[i]["exp_avg"] for i in range(n)])
    varr = _lib.tensor_array([opt.state[i]["exp_avg_sq"] for i in range(n)])
    carr = _lib.tensor_array(opt.working_copies)
    consts = (_lib.ElyConsts * n)()
    for j in range(n):
        consts[j].c[:] = optim.host_consts(LR, BETAS, EPS, WD, 2.0)
    aws = torch.empty(L.ely_adamw_workspace_bytes(n), dtype=torch.uint8, device=device)

    def fused(_):
        _lib.check(L.ely_adamw_fold_step(parr, aarr, garr, marr, varr, carr, n, consts, _lib.ORDER_HOST, 1, None, aws.data_ptr(), aws.numel(), sptr), "fold step")

    def fold_then_step(_):
        for a, g in zip(accs, grads):
            _lib.check(L.ely_fold_add(a.data_ptr(), g.data_ptr(), _lib.BF16, a.numel(), sptr), "fold")
        _lib.check(L.ely_adamw_step(parr, aarr, marr, varr, carr, n, consts, _lib.ORDER_HOST, 1, None, aws.data_ptr(), aws.numel(), sptr), "step")

    fused_ms = time_events(fused, iters, stream)
    unfused_ms = time_events(fold_then_step, iters, stream)
    del opt, params, grads, accs
    return {
        "fused_ms": fused_ms,
        "fused_GBs": n_elem * 32 / fused_ms / 1e6,
        "fold_then_step_ms": unfused_ms,
        "saved_frac": 1.0 - fused_ms / unfused_ms,
    }


def bench_tied_fold(device, stream, n_mb: int = 8, n_rows: int = 32768, rows_per_mb: int = 4096, iters: int = 3):
    """The tied table's row fold (accumulate.TiedRowFold, the drop-in for
    runtime/accumulate.py:140-247) on the Head of C1's model: a 32,768-row
    table (the reference presets' vocabulary, model/gpt.py:257-266) at
    d = 2560 in fp32, 8 microbatches each touching 4,096 random rows, the
    embedding rows arriving one microbatch behind the Head gradients.
    Against the stock dense fold in torch ops (e_i scattered into a dense
    zero table, g_i = h_i + e_i, acc = g_0 then acc += g_i); both are timed
    between HIP events over the whole fold and must agree bit for bit."""
    from elysium_wan_amd.accumulate import TiedRowFold

    d = D_MODEL
    gen = torch.Generator(device=device).manual_seed(21)
    hs = [torch.randn(n_rows, d, device=device, generator=gen) * 1e-3 for _ in range(n_mb)]
    rows = [torch.randperm(n_rows, device=device, generator=gen)[:rows_per_mb].sort().values.cpu() for _ in range(n_mb)]
    es = [torch.randn(rows_per_mb, d, device=device, generator=gen) * 1e-3 for _ in range(n_mb)]

    def row_fold():
        fold = TiedRowFold(n_rows, range(n_mb))
        for mb in range(n_mb):
            fold.add_head(mb, hs[mb], rows[mb])
            if mb:
                fold.add_embed(mb - 1, es[mb - 1])
        fold.add_embed(n_mb - 1, es[n_mb - 1])
        return fold.result()

    def dense_fold():
        acc = None
        for mb in range(n_mb):
            e = torch.zeros(n_rows, d, device=device)
            e[rows[mb].to(device)] = es[mb]
            g = hs[mb] + e
            acc = g if acc is None else acc.add_(g)
        return acc

    def timed(fn):
        out = fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(iters):
            out = fn()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / iters, out

    t_row, a = timed(row_fold)
    t_dense, b = timed(dense_fold)
    same = bool(torch.equal(a.view(torch.int32), b.view(torch.int32)))
    # compulsory traffic: each h read once (4 B/elem), the sum written once per
    # microbatch and read back from the second on (4 + 4), the embedding rows once
    nbytes = n_rows * d * (8 + 12 * (n_mb - 1)) + n_mb * rows_per_mb * d * 4
    del hs, es, a, b
    return {"rows": n_rows, "d": d, "microbatches": n_mb, "rows_per_mb": rows_per_mb, "row_fold_ms": t_row,
            "dense_fold_ms": t_dense, "row_fold_GBs": nbytes / (t_row * 1e-3) / 1e9, "bits_equal": same}


def bench_release(device, stream, tokens: int = 2048, iters: int = 3, moments: str = "device"):
    """Per-layer release (runtime/stage.py:3080-3099, RUNTIME-I23): the C1
    step runs on a side stream with on_param recording one event per block
    (12 tensors) as its update group is issued, while a forward-style
    consumer on the caller's stream waits on each block's event and then
    multiplies a [tokens, d] bf16 activation by that block's four bf16
    working-copy matrices.  Against: the single-launch step, then the same
    forward after it.  Reported: time from the step's start to block 0's
    release and to the last block's, and the wall time of step + forward
    both ways (HIP events).  moments="host" runs the "adamw-host" recipe's
    memory contract (moments in pinned host memory, updated in place over
    PCIe), the case the reference built the release for, with one
    iteration."""
    from elysium_wan_amd import optim

    params, grads = make_shard(device)
    per_block = len(block_shapes(D_MODEL))
    opt = optim.FusedAdamW(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order="host", max_norm=MAX_NORM,
                           working_copy=True, moments=moments,
                           release_elems=12 * D_MODEL * D_MODEL + 13 * D_MODEL)  # one group per block
    copies = opt.working_copies
    x = torch.randn(tokens, D_MODEL, device=device).bfloat16()
    side = torch.cuda.Stream(device)
    linear = torch.nn.functional.linear

    def forward(block, s):
        """One block's four GEMMs on its bf16 working copies (qkv, proj,
        fc1, fc2 at positions 2, 4, 8, 10 of the block's tensors)."""
        w = lambda j: copies[block * per_block + j]  # noqa: E731
        with torch.cuda.stream(s):
            h = linear(x, w(2))[:, :D_MODEL].contiguous()
            h = linear(h, w(4))
            h = linear(h, w(8))
            return linear(h, w(10))

    def serial():
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        opt.step(grads=grads)
        for b in range(N_BLOCKS):
            forward(b, stream)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end)

    def overlapped():
        """The reference's overlapped step (runtime/stage.py:3094-3099): the
        step on a side thread and stream, the forward on this thread waiting
        for each block's event as the side thread records it."""
        import threading

        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        events = [None] * N_BLOCKS
        ready = [threading.Event() for _ in range(N_BLOCKS)]
        left = [per_block] * N_BLOCKS
        start.record(stream)
        side.wait_stream(stream)

        def release(i):
            b = i // per_block
            left[b] -= 1
            if left[b] == 0:
                ev = torch.cuda.Event(enable_timing=True)
                ev.record(side)
                events[b] = ev
                ready[b].set()

        def run_step():
            torch.cuda.set_device(device)
            with torch.cuda.stream(side):
                opt.step(grads=grads, on_param=release)

        t = threading.Thread(target=run_step)
        t.start()
        for b in range(N_BLOCKS):
            ready[b].wait()
            stream.wait_event(events[b])
            forward(b, stream)
        end.record(stream)
        t.join()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        return start.elapsed_time(end), start.elapsed_time(events[0]), start.elapsed_time(events[-1])

    serial()
    overlapped()
    ser = [serial() for _ in range(iters)]
    ovl = [overlapped() for _ in range(iters)]
    fwd_start, fwd_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fwd_start.record(stream)
    for b in range(N_BLOCKS):
        forward(b, stream)
    fwd_end.record(stream)
    torch.cuda.synchronize()
    del opt, params, grads, copies
    return {
        "moments": moments,
        "forward_tokens": tokens,
        "forward_alone_ms": fwd_start.elapsed_time(fwd_end),
        "serial_step_then_forward_ms": min(ser),
        "per_layer_release_ms": min(o[0] for o in ovl),
        "first_block_released_ms": min(o[1] for o in ovl),
        "last_block_released_ms": min(o[2] for o in ovl),
    }


def bench_elementwise(device, stream, iters=5):
    """The stand-alone passes of the unfused path over C1's 192-tensor shard,
    one launch per tensor as the reference's callers make them: the fp32 ->
    bf16 working-copy cast (pieces.cast_piece, 6 B/elem), the first term of
    the fold widened to fp32 (pieces.fold_start, 6 B/elem), the fold of a bf16
    microbatch gradient into its fp32 sum (pieces.fold_add, 10 B/elem),
    the in-place scale of bf16 gradients by a device coefficient
    (ely_scale_inplace over the list, one launch per 48 tensors, 4 B/elem)
    and clip_grad_norm_ in one call (the norm, then one launch scaling every
    gradient: 6 B/elem)."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    sptr = _lib.stream_ptr(device)
    params, grads = make_shard(device)
    n = sum(p.numel() for p in params)
    copies = [torch.empty(p.shape, dtype=torch.bfloat16, device=device) for p in params]
    accs = [torch.zeros_like(p) for p in params]
    wide = [torch.empty_like(p) for p in params]
    garr = _lib.tensor_array(grads)
    one = torch.ones(1, dtype=torch.float32, device=device)

    def cast(_):
        for p, c in zip(params, copies):
            _lib.check(L.ely_cast_bf16(p.data_ptr(), c.data_ptr(), p.numel(), sptr), "cast")

    def fold(_):
        for a, g in zip(accs, grads):
            _lib.check(L.ely_fold_add(a.data_ptr(), g.data_ptr(), _lib.BF16, a.numel(), sptr), "fold")

    def widen(_):
        for w, g in zip(wide, grads):
            _lib.check(L.ely_widen_bf16(g.data_ptr(), w.data_ptr(), w.numel(), sptr), "widen")

    def scale(_):
        _lib.check(L.ely_scale_inplace(garr, len(grads), one.data_ptr(), sptr), "scale")

    res = torch.zeros(16, dtype=torch.uint8, device=device)
    nws = _lib.workspace(device, L.ely_grad_norm_workspace_bytes(garr, len(grads)))

    def clip(_):
        # clip_grad_norm_ in one call: the norm (2 B/elem) and one launch scaling every gradient (4 B/elem)
        _lib.check(L.ely_grad_norm_clip(garr, len(grads), MAX_NORM, res.data_ptr(), nws.data_ptr(), nws.numel(), sptr), "clip")

    out = {}
    for name, fn, b in (("cast_bf16", cast, 6), ("widen_bf16", widen, 6), ("fold_add_bf16", fold, 10), ("scale_bf16", scale, 4),
                        ("clip_grad_norm_bf16", clip, 6)):
        ms = time_events(fn, iters, stream)
        out[name] = {"ms": ms, "GBs": n * b / ms / 1e6}
    del params, grads, copies, accs, wide
    return out


def bench_host_moments(device, steps=3):
    """adamw-host with its moments in pinned host memory (the reference's
    recipe), updated in place through the GPU's mapping of the pinned
    buffers, and, for comparison, streamed through HBM in 2^24-element chunks
    over 3 staging slots (the reference's scheme): the PCIe-inclusive rate of
    C1's step (m and v cross PCIe both ways, 16 B per element), against the
    HBM-resident `value`."""
    from elysium_wan_amd import optim

    params, grads = make_shard(device)
    n_elem = sum(p.numel() for p in params)
    out = {}
    for name, pipeline in (("in_place", None), ("staged", True)):
        opt = optim.FusedAdamW(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order="host", max_norm=MAX_NORM,
                               working_copy=True, moments="host", pipeline=pipeline)
        opt.step(grads=grads)
        t0 = time.perf_counter()
        for _ in range(steps):
            opt.step(grads=grads)  # synchronizes at its end, as the reference's does
        dt = (time.perf_counter() - t0) / steps
        out[name] = {"step_s": dt, "params_per_s": n_elem / dt, "pcie_GBs": n_elem * 16 / dt / 1e9}
        if pipeline:
            # one more staged step with HIP events around every chunk copy on
            # its own stream (the step's time above is taken without them)
            opt.copy_timing = []
            opt.step(grads=grads)
            out[name]["copies"] = _copy_event_summary(opt.copy_timing)
            opt.copy_timing = None
        del opt
        torch.cuda.empty_cache()
    del params, grads
    return out


def _copy_event_summary(events) -> dict:
    """Per direction: count, median / min / max duration (ms) and the median
    rate of the staged step's chunk copies, from their HIP event pairs."""
    out = {}
    for what in ("h2d", "d2h"):
        ms = sorted(e0.elapsed_time(e1) for w, e0, e1 in events if w == what)
        if not ms:
            continue
        med = ms[len(ms) // 2]
        out[what] = {"count": len(ms), "median_ms": med, "min_ms": ms[0], "max_ms": ms[-1],
                     "slower_than_3ms": sum(1 for x in ms if x > 3.0),
                     "median_GBs": (1 << 24) * 4 / med / 1e6}
    return out


# benchmarks/wan/runs/2026-10-12-sxm4/REPORT.md:23-29: check_host_adamw.py's
# seconds per step at 200M parameters on an H100 80GB SXM host (the only
# published figures for this path)
REF_HOST_ADAMW_200M_S = {"serial": 0.074, "staged": 0.045, "staged_half_resident": 0.024}


def bench_check_host_adamw(device, params_m: float = 200.0, steps: int = 3):
    """benchmarks/wan/check_host_adamw.py:58-80 on this build: "adamw-host"
    (the reference's memory contract, moments in pinned host memory) over
    params_m million fp32 parameters in four tensors, fp32 grads N(0, 1),
    seconds per step of each arm -- serial copies, staged copies (the
    reference's default), staged with half the moments promoted to the GPU,
    and this build's default, the in-place update through the GPU's mapping
    (alone and with half resident) -- beside the reference's published
    figures."""
    from elysium_wan_amd import optim

    n = int(params_m * 1e6)
    out = {"params_m": params_m, "reference_h100_sxm_s": REF_HOST_ADAMW_200M_S if params_m == 200.0 else None}
    arms = (("serial", False, 0.0), ("staged", True, 0.0), ("staged_half_resident", True, 0.5),
            ("in_place", None, 0.0), ("in_place_half_resident", None, 0.5))
    for name, pipeline, resident in arms:
        gen = torch.Generator(device=device).manual_seed(2)
        params = [torch.empty(s, device=device).normal_(generator=gen).requires_grad_(True)
                  for s in (n // 4, n // 4, n // 2 - 7, 7)]
        for p in params:
            p.grad = torch.randn_like(p)
        opt = optim.build("adamw-host", params, 3e-4, pipeline=pipeline)
        opt.step()  # allocates the host moments
        if resident:
            opt.promote(int(resident * 8 * n))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            opt.step()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        out[name] = {"step_s": dt, "pcie_GBs": 16 * n * (1.0 - resident) / dt / 1e9}
        del params, opt
        torch.cuda.empty_cache()
    return out


def cpu_baseline(sample_elems: int, threads: int, target_s: float = 10.0, max_steps: int = 50):
    """The reference's CPU path for the same step, timed on this host's cores:
    torch.nn.utils.clip_grad_norm_ (foreach=False), torch.optim.AdamW
    (foreach=False; the "adamw" recipe, runtime/optim.py:50-51, on the CPU)
    and the bf16 working copy (pieces.cast_piece, runtime/pieces.py:192-195)
    over a prefix of C1's shard: fp32 params N(0, 0.02), the bf16 grads
    N(0, 1e-4) widened to fp32 beforehand (pieces.fold_start), as many steps
    as fit `target_s` seconds.  -> (params/s, seconds, steps)."""
    threads0 = torch.get_num_threads()
    try:
        gen = torch.Generator().manual_seed(0)
        p = (torch.randn(sample_elems, generator=gen) * 0.02).requires_grad_(True)
        p.grad = (torch.randn(sample_elems, generator=gen) * 1e-4).bfloat16().float()
        copy = torch.empty(sample_elems, dtype=torch.bfloat16)
        torch.set_num_threads(threads)
        opt = torch.optim.AdamW([p], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, foreach=False)

        def step():
            torch.nn.utils.clip_grad_norm_([p], MAX_NORM, foreach=False)
            opt.step()
            copy.copy_(p.detach())

        step()  # moments allocated; first-touch page faults outside the timed steps
        t0 = time.perf_counter()
        k = 0
        while k < max_steps and (k < 2 or time.perf_counter() - t0 < target_s):
            step()
            k += 1
        dt = time.perf_counter() - t0
        del opt, p, copy
        return sample_elems * k / dt, dt, k
    finally:
        torch.set_num_threads(threads0)


def cpu_port_baseline(sample_elems: int, steps: int = 2):
    """The oracle's HostAdamW (one thread of C) over a prefix of C1's shard."""
    from oracle import oracle as O

    rng = np.random.default_rng(0)
    block = 1 << 22
    reps = -(-sample_elems // block)
    p = np.tile((rng.standard_normal(block) * 0.02).astype(np.float32), reps)[:sample_elems]
    g = np.tile(O.f32_to_bf16_bits((rng.standard_normal(block) * 1e-4).astype(np.float32)), reps)[:sample_elems]
    m = np.zeros(sample_elems, np.float32)
    v = np.zeros(sample_elems, np.float32)
    cp = np.zeros(sample_elems, np.uint16)
    t0 = time.perf_counter()
    for s in range(steps):
        O.adamw_host(p, g, m, v, O.host_adamw_consts(LR, BETAS, EPS, WD, s + 1), True, 1.0, cp)
    dt = time.perf_counter() - t0
    return sample_elems * steps / dt, dt


def profile_pass(device):
    """A short run of every kernel bench.py measures, for rocprofv3 --pmc
    passes (one counter set per run): a plain streaming kernel of known size
    (the fp32 -> bf16 cast of 2^28 elements: reads 1 GiB, writes 512 MiB)
    to calibrate the counters, three optimizer steps over C1's shard and
    three quantize / dequantize launches of C1's activation."""
    from elysium_wan_amd import _lib, optim

    L = _lib.load()
    sptr = _lib.stream_ptr(device)
    x = torch.empty(CAL_ELEMS, dtype=torch.float32, device=device).normal_()
    y = torch.empty(CAL_ELEMS, dtype=torch.bfloat16, device=device)
    for _ in range(3):
        _lib.check(L.ely_cast_bf16(x.data_ptr(), y.data_ptr(), CAL_ELEMS, sptr), "cast")
    torch.cuda.synchronize()
    del x, y
    log("profile pass: calibration done")
    params, grads = make_shard(device)
    opt = optim.FusedAdamW(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, order="host", max_norm=MAX_NORM, working_copy=True)
    for _ in range(3):
        opt.step(grads=grads)
    torch.cuda.synchronize()
    del opt, params, grads
    log("profile pass: optimizer done")
    rows, cols = 8 * 2048, D_MODEL
    xa = torch.randn(rows, cols, device=device).to(torch.bfloat16)
    q = torch.empty(rows, cols, dtype=torch.uint8, device=device)
    k = torch.empty(rows, dtype=torch.int32, device=device)
    out = torch.empty(rows, cols, dtype=torch.bfloat16, device=device)
    ws = _lib.workspace(device, L.ely_fp8_workspace_bytes(rows, cols, _lib.BF16))
    for _ in range(3):
        _lib.check(L.ely_fp8_quantize(xa.data_ptr(), _lib.BF16, rows, cols, _lib.E4M3, q.data_ptr(), k.data_ptr(), ws.data_ptr(), ws.numel(), sptr), "q")
        _lib.check(L.ely_fp8_dequantize(q.data_ptr(), k.data_ptr(), rows, cols, _lib.E4M3, out.data_ptr(), _lib.BF16, sptr), "dq")
    torch.cuda.synchronize()
    del xa, q, k, out
    log("profile pass: codec done")
    # per-tensor quantize of a C4-sized activation with a right exponent hint
    # (one pass: quant_hint_kernel), after one call without a hint that finds
    # k (the sampled guess, whose hint pass on this N(0, 1) input is right too)
    n4 = 16 * 4096 * 8192
    x4 = torch.randn(n4, device=device).to(torch.bfloat16)
    q4 = torch.empty(n4, dtype=torch.uint8, device=device)
    k4 = torch.empty(1, dtype=torch.int32, device=device)
    ws = _lib.workspace(device, max(L.ely_fp8_workspace_bytes(1, n4, _lib.BF16), L.ely_fp8_hint_workspace_bytes(n4)))
    _lib.check(L.ely_fp8_quantize(x4.data_ptr(), _lib.BF16, 1, n4, _lib.E4M3, q4.data_ptr(), k4.data_ptr(), ws.data_ptr(), ws.numel(), sptr), "q")
    hint = int(k4.item())
    for _ in range(3):
        _lib.check(L.ely_fp8_quantize_hint(x4.data_ptr(), _lib.BF16, n4, _lib.E4M3, hint, None, q4.data_ptr(), k4.data_ptr(), None,
                                           None, ws.data_ptr(), ws.numel(), sptr), "qh")
    torch.cuda.synchronize()
    log("profile pass: per-tensor hint done")


# Kernels the traffic summary reports: name fragment -> (algorithmic bytes per
# launch, what they are).  C1 sizes.
def _traffic_kernels():
    n = sum(int(np.prod(s)) for s in block_shapes(D_MODEL)) * N_BLOCKS
    act = 8 * 2048 * D_MODEL
    return {
        "adamw_kernel": (n * ADAM_BYTES_PER_ELEM, "fused clip + AdamW, C1 shard, 28 B/elem"),
        "norm_partials_kernel": (n * NORM_BYTES_PER_ELEM, "grad-norm partials, C1 bf16 grads, 2 B/elem"),
        "quant_rows_kernel": (act * CODEC_BYTES_PER_ELEM, "fp8 e4m3 quantize, C1 activation, 3 B/elem"),
        "dequant_flat_kernel": (act * CODEC_BYTES_PER_ELEM, "fp8 e4m3 dequantize -> bf16, C1 activation, 3 B/elem"),
        "quant_hint_kernel": (16 * 4096 * 8192 * CODEC_BYTES_PER_ELEM,
                              "fp8 e4m3 per-tensor quantize with a right hint, C4 activation, 3 B/elem"),
    }


def _pmc_means(directory: str, counter: str) -> dict:
    """Mean per-dispatch value of `counter` for each kernel name in a
    rocprofv3 --pmc output directory (every *counter_collection.csv under it)."""
    import csv
    import glob

    sums: dict = {}
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    for path in files:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                name = row["Kernel_Name"]
                s = sums.setdefault(name, [0.0, 0])
                s[0] += float(row["Counter_Value"])
                s[1] += 1
    return {name: v[0] / v[1] for name, v in sums.items()}


def _pick(means: dict, fragment: str):
    hits = [v for name, v in means.items() if fragment in name]
    if not hits:
        return None
    return sum(hits) / len(hits)


READ_SIZE_COUNTERS = ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_sum")


def traffic_summary(fetch_dir: str, write_dir: str, command: str, sizes_dir: str | None = None) -> None:
    """HBM bytes per launch of each measured kernel from two rocprofv3 --pmc
    runs of `bench.py --profile-pass` (FETCH_SIZE, then WRITE_SIZE; KiB per
    dispatch), each scaled by the same counter's reading on the calibration
    cast (known: 4 B read + 2 B written per element).  The read factor is
    cross-checked on the read-only grad-norm kernel (known: 2 B per bf16
    gradient), and, with a third run of the request-size counters
    (READ_SIZE_COUNTERS), by the bytes the read requests of each size carry.
    Writes profiles/adamw_c1_traffic.json (read back by bench.py) and a text
    summary beside it."""
    fetch = _pmc_means(fetch_dir, "FETCH_SIZE")
    write = _pmc_means(write_dir, "WRITE_SIZE")
    cf = _pick(fetch, "cast_bf16_kernel") * 1024.0 / (CAL_ELEMS * 4)
    cw = _pick(write, "cast_bf16_kernel") * 1024.0 / (CAL_ELEMS * 2)
    out = {"fetch_factor": cf, "write_factor": cw, "command": command, "kernels": {}}
    lines = [
        "# HBM traffic per launch (rocprofv3 --pmc), C1 workload and C4's per-tensor hint path",
        "",
        f"Command: `{command}`",
        "",
        f"Calibration: cast_bf16_kernel over {CAL_ELEMS} fp32 -> bf16 (reads {CAL_ELEMS * 4} B, writes {CAL_ELEMS * 2} B);",
        f"FETCH_SIZE reads {cf:.4f} x the known bytes, WRITE_SIZE {cw:.4f} x.  Every figure below is divided by these factors.",
        "",
        *_read_factor_checks(fetch, sizes_dir, cf),
        "",
        "| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic (B) | algorithmic (B) | traffic / algorithmic | what |",
        "|---|---|---|---|---|---|---|",
    ]
    for frag, (alg, what) in _traffic_kernels().items():
        fk, wk = _pick(fetch, frag), _pick(write, frag)
        if fk is None or wk is None:
            continue
        t = fk * 1024.0 / cf + wk * 1024.0 / cw
        out["kernels"][frag] = {"fetch_kib": fk, "write_kib": wk, "traffic_bytes": t, "algorithmic_bytes": alg, "ratio": t / alg}
        lines.append(f"| {frag} | {fk:.0f} | {wk:.0f} | {t:.4g} | {alg:.4g} | {t / alg:.3f} | {what} |")
    adam = out["kernels"].get("adamw_kernel")
    out["traffic_bytes_per_launch"] = adam["traffic_bytes"] if adam else None
    nk = _pick(fetch, "norm_partials_kernel")
    if nk is not None:
        out["norm_raw_fetch_factor"] = nk * 1024.0 / _traffic_kernels()["norm_partials_kernel"][0]
    os.makedirs(os.path.join(HERE, "profiles"), exist_ok=True)
    with open(os.path.join(HERE, "profiles", "adamw_c1_traffic.json"), "w") as f:
        json.dump(out, f, indent=1)
    with open(os.path.join(HERE, "profiles", "adamw_c1_traffic.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def _read_factor_checks(fetch: dict, sizes_dir: str | None, cf: float) -> list:
    """Lines of the traffic summary that cross-check the FETCH_SIZE factor:
    the read-only grad-norm kernel's raw reading against its known bytes,
    and, from a run of READ_SIZE_COUNTERS, the bytes the read requests carry
    (32 x 32-byte + 64 x 64-byte + 128 x 128-byte requests) against
    FETCH_SIZE for the same kernels."""
    lines = ["Cross-checks of the read factor:", ""]
    nk = _pick(fetch, "norm_partials_kernel")
    if nk is not None:
        known = _traffic_kernels()["norm_partials_kernel"][0]
        lines.append(f"- norm_partials_kernel, read-only, known {known} B read: raw FETCH_SIZE / known = "
                     f"{nk * 1024.0 / known:.4f} (calibration cast: {cf:.4f})")
    if sizes_dir:
        m = {c: _pmc_means(sizes_dir, c) for c in READ_SIZE_COUNTERS}
        for frag, known in (("cast_bf16_kernel", CAL_ELEMS * 4), ("norm_partials_kernel", _traffic_kernels()["norm_partials_kernel"][0]),
                            ("adamw_kernel", None)):
            r32, r64, r128, rall = (_pick(m[c], frag) for c in READ_SIZE_COUNTERS)
            if rall is None:
                continue
            b = 32 * (r32 or 0) + 64 * (r64 or 0) + 128 * (r128 or 0)
            fk = _pick(fetch, frag)
            txt = (f"- {frag}: {rall:.4g} read requests, {r128 or 0:.4g} of 128 B, {r64 or 0:.4g} of 64 B, {r32 or 0:.4g} of 32 B; "
                   f"they carry {b:.4g} B")
            if known:
                txt += f" = {b / known:.4f} x the known {known} B"
            if fk:
                txt += f"; FETCH_SIZE counts {fk * 1024.0 / b:.4f} x that"
            lines.append(txt)
    return lines


def _dispatches(trace_dir: str):
    """(kernel name, duration ns) of every dispatch in a rocprofv3
    --kernel-trace csv directory, in dispatch order."""
    import csv
    import glob

    rows = []
    for path in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        with open(path) as f:
            rows += list(csv.DictReader(f))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return [(r["Kernel_Name"], int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) for r in rows]


def _runs(disp, names):
    """Maximal runs of consecutive dispatches of one of `names` (other kernels
    in between end a run) -> [(name, [durations])]."""
    runs = []
    for name, ns in disp:
        if name not in names:
            if runs and runs[-1][0] is not None:
                runs.append((None, []))
            continue
        if runs and runs[-1][0] == name:
            runs[-1][1].append(ns)
        else:
            runs.append((name, [ns]))
    return [r for r in runs if r[0] is not None]


def _c1_codec_labels(fmts: int = 2) -> list:
    """(kind, mode) of every quant_rows_kernel / dequant_flat_kernel launch of
    `bench.py --no-optimizer --codec c1`, in launch order: per format,
    bench_codec's warm-up quantizes, then time_events of quantize,
    dequantize and the round trip, then time_back_to_back of the three; each
    timed group opens with one untimed launch."""
    labels = []
    for _ in range(fmts):
        labels += [("quantize", "warm")] * C1_CODEC_COPIES
        for mode in ("single", "b2b"):
            for kind in ("quantize", "dequantize", "roundtrip"):
                labels += [(kind, "untimed")] + [(kind, mode)] * C1_CODEC_ITERS
    return labels


def _codec_calls(disp) -> list:
    """Group a codec trace's dispatches into calls: (kind, [(kernel, ns)])
    with kind "row" (one quant_rows / quant_block_row kernel: a per-row
    quantize or round trip), "deq" (a dequantize), "guess" (a per-tensor
    quantize or round trip without a hint: guess_amax, sample_max, then the
    hint path's three kernels), "split" (the split path's row maxima and
    quant_split_kernel) or "hint" (ely_fp8_quantize_hint's three kernels).
    Other kernels (torch's) are skipped."""
    calls, cur, kind = [], [], None
    ends = {"guess": "quant_hint_fixup_kernel", "hint": "quant_hint_fixup_kernel", "split": "quant_split_kernel"}
    for name, ns in disp:
        if kind is not None:
            cur.append((name, ns))
            if name == ends[kind]:
                calls.append((kind, cur))
                cur, kind = [], None
            continue
        if name in ("quant_rows_kernel", "quant_block_row_kernel"):
            calls.append(("row", [(name, ns)]))
        elif name.startswith("dequant_"):
            calls.append(("deq", [(name, ns)]))
        elif name == "guess_amax_kernel":
            cur, kind = [(name, ns)], "guess"
        elif name == "rowmax_partial_kernel":
            cur, kind = [(name, ns)], "split"
        elif name == "quant_hint_kernel":
            cur, kind = [(name, ns)], "hint"
    return calls


def _c4_labels() -> list:
    """(scaling, op, mode) of every codec call of `bench.py --no-optimizer
    --codec c4`, in launch order: per input (activation, gradient), scaling
    (per-row, per-tensor) and format, bench_codec's two warm-up quantizes,
    then quantize, dequantize and round trip timed one call between two
    HIP events (each group after one untimed call), the per-tensor hint
    calls (11 right, 11 one off, 11 round trips with the right hint, one
    more right), then the stats pass's quantize and dequantize."""
    labels = []
    for _ in ("activation", "gradient"):
        for sc in ("per-row", "per-tensor"):
            for _f in ("e4m3", "e5m2"):
                labels += [(sc, "quantize", "warm")] * 2
                for op in ("quantize", "dequantize", "round trip"):
                    labels += [(sc, op, "untimed")] + [(sc, op, "timed")] * C4_CODEC_ITERS
                if sc == "per-tensor":
                    labels += [(sc, "hint right", "untimed")] + [(sc, "hint right", "timed")] * C4_CODEC_ITERS
                    labels += [(sc, "hint off", "untimed")] + [(sc, "hint off", "timed")] * C4_CODEC_ITERS
                    labels += [(sc, "hint round trip", "untimed")] + [(sc, "hint round trip", "timed")] * C4_CODEC_ITERS
                    labels += [(sc, "hint right", "extra")]
                labels += [(sc, "quantize", "stats"), (sc, "dequantize", "stats")]
    return labels


def c4_summary(trace_dir: str, bench_out: str | None) -> None:
    """Kernel durations of a rocprofv3 --kernel-trace run of `bench.py
    --no-optimizer --codec c4`, the calls labelled by bench_codec's launch
    order (_c4_labels), averaged over both inputs and formats over the
    timed calls.  A per-tensor call is its kernels added up.  Writes
    profiles/codec_c4_kernel_trace.md."""
    calls = _codec_calls(_dispatches(trace_dir))
    labels = _c4_labels()
    if len(calls) < len(labels):
        raise SystemExit(f"the C4 trace holds {len(calls)} codec calls, bench_codec makes {len(labels)}")
    want = {"dequantize": ("deq",), "quantize": ("row", "guess", "split"), "round trip": ("row", "guess", "split"),
            "hint right": ("hint", "split"), "hint off": ("hint", "split"), "hint round trip": ("hint", "split")}
    timed = {}  # (scaling, op) -> [total ns per call]
    parts = {}  # (scaling, op, kernel) -> [ns]
    kinds = {}  # (scaling, op) -> call kinds seen
    for (sc, op, mode), (kind, ks) in zip(labels, calls):
        if kind not in want[op]:
            raise SystemExit(f"codec call {kind} where bench_codec's order has {sc} {op}")
        if mode != "timed":
            continue
        timed.setdefault((sc, op), []).append(sum(ns for _, ns in ks))
        kinds.setdefault((sc, op), set()).add(kind)
        if sc == "per-tensor":
            for k, ns in ks:
                parts.setdefault((op, k), []).append(ns)
    n = 16 * 4096 * 8192
    per = {"quantize": 3, "dequantize": 3, "round trip": 4, "hint right": 3, "hint off": 3, "hint round trip": 4}
    lines = [
        "# Kernel durations, fp8 codec on C4's tensors",
        "",
        "Commands (on one MI355X, from the repository root):",
        "",
        "    rocprofv3 --kernel-trace --stats -T -d <dir> -o c4 --output-format csv -- python3 bench.py --no-optimizer --codec c4 > <run's stdout>",
        "    python bench.py --c4-summary <dir> --bench-json <run's stdout>",
        "",
        f"Workload: config C4's bf16 activation and gradient [16, 4096, 8192] ({n:,} elements,",
        "1.07 GB each; Student-t(3) with 0.01 % +-1e4 outliers, and N(0, 1e-5)), e4m3 and",
        "e5m2, per-row (8,192-wide rows) and per-tensor scaling, two copies of each",
        "input rotating.  Algorithmic bytes per element: 3 for quantize and",
        "dequantize, 4 for the fused round trip.  Each call is labelled by",
        "bench_codec's launch order; the figures are its timed calls (one call",
        f"between two HIP events, {C4_CODEC_ITERS} per group), averaged over both inputs",
        "and formats, a call's kernels added up.",
        "",
        "A per-tensor quantize or round trip with no hint guesses the exponent",
        "from the |x|max of every 61st 2,048-element segment (guess_amax_kernel,",
        "sample_max_kernel) and runs the hint path at the guess: quant_hint_kernel",
        "converts at the guess while it reduces each segment's |x|max,",
        "hint_reduce_kernel folds those, and quant_hint_fixup_kernel exits when",
        "the tensor's exponent equals the guess, or converts every segment again",
        "(a second read of x) when it does not.",
        "",
        "| scaling | operation | calls | average (µs) | algorithmic rate | fraction of 8 TB/s |",
        "|---|---|---|---|---|---|",
    ]
    names = {"hint right": "quantize, right hint (`k_hint`)", "hint off": "quantize, hint off by one",
             "hint round trip": "round trip, right hint"}
    for sc in ("per-row", "per-tensor"):
        for op in ("quantize", "dequantize", "round trip", "hint right", "hint off", "hint round trip"):
            ds = timed.get((sc, op))
            if not ds:
                continue
            avg = sum(ds) / len(ds)
            rate = n * per[op] / avg / 1e3
            lines.append(f"| {sc} | {names.get(op, op)} | {len(ds)} | {avg / 1e3:,.1f} | {rate:.2f} TB/s | {rate / 8:.2f} |")
    if parts:
        lines += ["", "Per-tensor calls by kernel (average µs over the timed calls):", "",
                  "| operation | kernel | calls | average (µs) |", "|---|---|---|---|"]
        order = ("quantize", "round trip", "hint right", "hint off", "hint round trip")
        for op in order:
            for (o, k), ds in parts.items():
                if o == op:
                    lines.append(f"| {names.get(op, op)} | {k} | {len(ds)} | {sum(ds) / len(ds) / 1e3:,.1f} |")
    b = None
    if bench_out:
        with open(bench_out) as f:
            rows = [ln for ln in f.read().splitlines() if ln.startswith('{"c4"')]
        b = json.loads(rows[-1])["c4"] if rows else None
    if b:
        lines += ["", "bench.py's HIP-event figures in the traced process (activation, e4m3):"]
        for sc, key in (("per-row", "per_row"), ("per-tensor", "per_tensor")):
            e = b["activation"][key]["e4m3"]
            lines.append(f"{sc}: quantize {e['quantize_GBs'] / 1e3:.2f} TB/s, dequantize {e['dequantize_GBs'] / 1e3:.2f} TB/s, "
                         f"round trip {e['roundtrip_GBs'] / 1e3:.2f} TB/s.")
    with open(os.path.join(HERE, "profiles", "codec_c4_kernel_trace.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def _row(label, ds):
    return f"| {label} | {len(ds)} | {sum(ds) / len(ds):,.0f} | {min(ds):,} | {max(ds):,} |"


def _last_bench_line(path: str | None):
    """The last bench.py JSON line in a file of that run's output (rocprofv3
    may print around it), or None.  A codec-only run's {"c1": ...} line is
    returned in the full line's shape ({"fp8_codec": {"c1_per_row": ...}})."""
    if not path:
        return None
    with open(path) as f:
        text = f.read().splitlines()
    rows = [ln for ln in text if ln.startswith('{"metric"')]
    if rows:
        return json.loads(rows[-1])
    rows = [ln for ln in text if ln.startswith('{"c1"')]
    return {"fp8_codec": {"c1_per_row": json.loads(rows[-1])["c1"]}} if rows else None


def trace_summary(step_dir: str, codec_dir: str, bench_json: list | None) -> None:
    """Kernel durations from two rocprofv3 --kernel-trace runs: the C1
    optimizer step (`bench.py --no-cpu --no-codec --no-extra`) and the C1
    codec (`bench.py --no-optimizer --codec c1`).  The codec's quantize and
    fused round trip are one kernel (quant_rows_kernel, with or without the
    dequantized output), told apart by bench_codec's launch order: per
    format, quantize launches, dequantize launches, then as many round trips
    as dequantizes.  Writes profiles/c1_step_kernel_trace.md and
    profiles/codec_c1_kernel_trace.md; with `bench_json` (the output files
    of the two traced runs themselves, step then codec) each summary sets
    the HIP-event figures of the process it traced beside the trace."""
    bench_json = list(bench_json or [])
    b = _last_bench_line(bench_json[0] if bench_json else None)
    bc = _last_bench_line(bench_json[1] if len(bench_json) > 1 else None)
    n = N_BLOCKS * (12 * D_MODEL * D_MODEL + 13 * D_MODEL)
    step = _dispatches(step_dir)
    by = {}
    for name, ns in step:
        by.setdefault(name, []).append(ns)
    lines = [
        "# Kernel durations, C1 optimizer step (the roofline kernel)",
        "",
        "Commands (on one MI355X, from the repository root):",
        "",
        "    rocprofv3 --kernel-trace --stats -T -d <step dir> -o kt --output-format csv -- python3 bench.py --no-cpu --no-codec --no-extra > <step run's stdout>",
        "    python bench.py --trace-summary <step dir> <codec dir> --bench-json <step run's stdout> <codec run's stdout>",
        "",
        "Workload: config C1's shard (16 GPT blocks at d = 2560, 192 tensors,",
        f"{n:,} fp32 params, bf16 grads N(0, 1e-4), bf16 working copy, AdamW",
        "lr 3e-4, betas 0.9/0.95, eps 1e-8, weight decay 0.1, clip 1.0): warmup and",
        "timed optimizer steps, then event-timed launches of each kernel.",
        "",
        "| kernel | calls | average (ns) | min (ns) | max (ns) |",
        "|---|---|---|---|---|",
    ]
    lines += [_row(k, by[k]) for k in ("adamw_kernel", "norm_partials_kernel", "norm_final_kernel") if k in by]
    if "adamw_kernel" in by:
        avg = sum(by["adamw_kernel"]) / len(by["adamw_kernel"]) / 1e6
        lines += ["", f"adamw_kernel: {n * ADAM_BYTES_PER_ELEM / 1e9:.2f} GB ({ADAM_BYTES_PER_ELEM} B/elem) / {avg:.3f} ms = "
                  f"{n * ADAM_BYTES_PER_ELEM / avg / 1e6:,.0f} GB/s, {n * ADAM_BYTES_PER_ELEM / avg / 1e6 / HBM_PEAK_GBS:.3f} of 8 TB/s."]
        if b:
            ev = b["kernels"]["adamw_ms"]
            lines += [f"bench.py's HIP-event average in the traced process: {ev:.3f} ms ({abs(avg - ev) / ev * 100:.1f} % apart)."]
    with open(os.path.join(HERE, "profiles", "c1_step_kernel_trace.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))

    labels = _c1_codec_labels()
    disp = [(name, ns) for name, ns in _dispatches(codec_dir) if name in ("quant_rows_kernel", "dequant_flat_kernel")]
    want = ["dequant_flat_kernel" if lab[0] == "dequantize" else "quant_rows_kernel" for lab in labels]
    if [name for name, _ in disp][: len(labels)] != want:
        raise SystemExit("the codec trace does not follow bench_codec's launch order")
    by = {}
    for (kind, mode), (_, ns) in zip(labels, disp):
        by.setdefault((kind, mode), []).append(ns)
    na = 8 * 2048 * D_MODEL
    per = {"quantize": 3, "dequantize": 3, "roundtrip": 4}
    lines = [
        "# Kernel durations, fp8 codec on C1's activation",
        "",
        "Commands (on one MI355X, from the repository root):",
        "",
        "    rocprofv3 --kernel-trace --stats -T -d <codec dir> -o kc --output-format csv -- python3 bench.py --no-optimizer --codec c1 > <codec run's stdout>",
        "    python bench.py --trace-summary <step dir> <codec dir> --bench-json <step run's stdout> <codec run's stdout>",
        "",
        "Workload: config C1's boundary activation [8, 2048, 2560] bf16 (N(0, 1) with",
        "0.1% of the elements x50), per-row scaling (one exponent per 2,560-element",
        "row), e4m3 and e5m2, rotating through 8 copies so that no launch reads from",
        f"the 256 MB MALL.  Algorithmic traffic per launch: {na:,} x 3 B = {na * 3 / 1e6:.1f} MB",
        f"for quantize and dequantize, x 4 B = {na * 4 / 1e6:.1f} MB for the fused round trip.",
        "quant_rows_kernel serves quantize and the round trip; each launch is",
        f"labelled by bench_codec's fixed order (per format: {C1_CODEC_COPIES} warm-up quantizes, then",
        f"quantize, dequantize and round trip timed one launch between two HIP events,",
        f"then the same three queued back to back; each timed group is {C1_CODEC_ITERS} launches",
        "after one untimed launch that follows a device synchronize).",
        "",
        "| launches | timed single launches | average (ns) | min (ns) | max (ns) | kernel-time rate | back-to-back launches | average (ns) | rate | every launch, warm-up and untimed included | average (ns) | rate |",
        "|---|---|---|---|---|---|---|---|---|---|---|---|",
    ]
    for kind in ("quantize", "dequantize", "roundtrip"):
        ev, bb = by.get((kind, "single"), []), by.get((kind, "b2b"), [])
        every = ev + bb + by.get((kind, "untimed"), []) + (by.get(("quantize", "warm"), []) if kind == "quantize" else [])
        if not ev or not bb:
            continue
        rate = lambda ds: na * per[kind] / (sum(ds) / len(ds)) / 1e3  # noqa: E731
        lines.append(f"| {kind} | {len(ev)} | {sum(ev) / len(ev):,.0f} | {min(ev):,} | {max(ev):,} | {rate(ev):.2f} TB/s | "
                     f"{len(bb)} | {sum(bb) / len(bb):,.0f} | {rate(bb):.2f} TB/s | {len(every)} | "
                     f"{sum(every) / len(every):,.0f} | {rate(every):.2f} TB/s |")
    if bc and bc.get("fp8_codec"):
        c = bc["fp8_codec"]["c1_per_row"]["e4m3"]
        lines += ["", "bench.py's HIP-event averages in the traced process, e4m3 (one launch between two events, so each also",
                  f"holds the launch's dispatch latency): quantize {c['quantize_ms'] * 1e3:.1f} us ({c['quantize_GBs'] / 1e3:.2f} TB/s),",
                  f"dequantize {c['dequantize_ms'] * 1e3:.1f} us ({c['dequantize_GBs'] / 1e3:.2f} TB/s), round trip "
                  f"{c['roundtrip_ms'] * 1e3:.1f} us ({c['roundtrip_GBs'] / 1e3:.2f} TB/s)."]
        b2b = c.get("back_to_back_GBs")
        if b2b:
            lines += [f"Back to back between one event pair: quantize {b2b['quantize'] / 1e3:.2f}, dequantize "
                      f"{b2b['dequantize'] / 1e3:.2f}, round trip {b2b['roundtrip'] / 1e3:.2f} TB/s."]
    with open(os.path.join(HERE, "profiles", "codec_c1_kernel_trace.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def bench_wire(device, stream, iters: int = 10):
    """The lossless boundary wires on C1's activation [8, 2048, 2560] bf16.
    The GPU half, between HIP events: the byte-plane split and join
    (4 B/elem), the e4m3 nibble encode (2 B read + 1 B written) and decode
    (1 B + 4 B fp32), and the scaled-fp8 wire's exponent recovery plus byte
    image in one call (ely_fp8_recover_image: 2 B read, 1 B written),
    rotating through 4 inputs.  Then the whole planes.encode / decode and
    encode_scaled_fp8 / decode calls (GPU half, the copy to the host and the
    host's zlib), wall-clock seconds."""
    from elysium_wan_amd import _lib, fp8

    L = _lib.load()
    sptr = _lib.stream_ptr(device)
    rows, cols = 8 * 2048, D_MODEL
    n = rows * cols
    copies = 4
    xs = _activations(device, rows, cols, copies, 11)
    planes = [torch.empty(2 * n, dtype=torch.uint8, device=device) for _ in range(copies)]
    back = [torch.empty(n, dtype=torch.bfloat16, device=device) for _ in range(copies)]
    out = {}
    ms = time_events(lambda i: _lib.check(L.ely_byteplanes_split(xs[i % copies].data_ptr(), n, 2, planes[i % copies].data_ptr(), sptr), "split"), iters, stream)
    out["byteplanes_split_GBs"] = 4 * n / ms / 1e6
    ms = time_events(lambda i: _lib.check(L.ely_byteplanes_join(planes[i % copies].data_ptr(), n, 2, back[i % copies].data_ptr(), sptr), "join"), iters, stream)
    out["byteplanes_join_GBs"] = 4 * n / ms / 1e6
    reps = [x.clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.bfloat16) for x in xs]  # e4m3-representable boundaries
    hi = [torch.empty((n + 1) // 2, dtype=torch.uint8, device=device) for _ in range(copies)]
    lo = [torch.empty((n + 1) // 2, dtype=torch.uint8, device=device) for _ in range(copies)]
    f32 = [torch.empty(n, dtype=torch.float32, device=device) for _ in range(2)]
    nbad = torch.zeros(1, dtype=torch.int64, device=device)
    ms = time_events(lambda i: _lib.check(L.ely_fp8_nibbles_encode(reps[i % copies].data_ptr(), _lib.BF16, n, hi[i % copies].data_ptr(), lo[i % copies].data_ptr(), nbad.data_ptr(), sptr), "nibbles"), iters, stream)
    out["nibbles_encode_GBs"] = 3 * n / ms / 1e6
    ms = time_events(lambda i: _lib.check(L.ely_fp8_nibbles_decode(hi[i % copies].data_ptr(), lo[i % copies].data_ptr(), n, f32[i % 2].data_ptr(), sptr), "nibbles"), iters, stream)
    out["nibbles_decode_GBs"] = 5 * n / ms / 1e6
    torch.cuda.synchronize()
    if int(nbad.item()):
        raise RuntimeError("bench_wire: an e4m3 cast was not e4m3-representable")
    del reps, hi, lo, f32
    bad = torch.zeros(1, dtype=torch.int64, device=device)
    rts = [fp8.roundtrip(x, "e4m3") for x in xs]
    ks = [torch.empty(rows, dtype=torch.int32, device=device) for _ in range(copies)]
    qs = [torch.empty(n, dtype=torch.uint8, device=device) for _ in range(copies)]
    ws = _lib.workspace(device, L.ely_fp8_recover_workspace_bytes(rows))

    def recover_and_image(i):
        j = i % copies
        _lib.check(L.ely_fp8_recover_image(rts[j].data_ptr(), _lib.BF16, rows, cols, _lib.E4M3, ks[j].data_ptr(), qs[j].data_ptr(),
                                           bad.data_ptr(), ws.data_ptr(), ws.numel(), sptr), "recover_image")

    ms = time_events(recover_and_image, iters, stream)
    out["scaled_fp8_image_GBs"] = 3 * n / ms / 1e6
    torch.cuda.synchronize()
    if int(bad.item()):
        raise RuntimeError("bench_wire: a recipe round trip was not recoverable")
    # the whole wire call as the reference's caller makes it (GPU half, the
    # copy to the host and the host's zlib), wall-clock seconds, one call
    from elysium_wan_amd import planes as _planes

    def wall(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        r = fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0, r

    _planes.encode(xs[0])  # warm: library load, thread pool
    secs, (payload, shape) = wall(lambda: _planes.encode(xs[0]))
    out["planes_encode_bf16_s"] = secs
    out["planes_decode_bf16_s"], _ = wall(lambda: _planes.decode(payload, shape))
    secs, (payload, shape) = wall(lambda: _planes.encode_scaled_fp8(rts[0], "e4m3"))
    out["scaled_fp8_encode_s"] = secs
    out["scaled_fp8_decode_s"], _ = wall(lambda: _planes.decode(payload, shape))
    del xs, planes, back, rts, ks, qs
    return out


def hbm_reference(device, stream, n: int = 1 << 28, iters: int = 10):
    """What the vendor stack itself reaches on this box for mixed read/write
    traffic, beside the analytic peak: torch's device-to-device copy_ of
    1 GiB (read 4 B + write 4 B per element) and torch.add(a, b, out=c)
    (read 8 B + write 4 B), HIP events on the bench stream."""
    a = torch.empty(n, device=device).normal_()
    b = torch.empty(n, device=device).normal_()
    c = torch.empty(n, device=device)
    copy_ms = time_events(lambda i: c.copy_(a), iters, stream)
    add_ms = time_events(lambda i: torch.add(a, b, out=c), iters, stream)
    del a, b, c
    return {"torch_copy_GBs": 8 * n / copy_ms / 1e6, "torch_add_GBs": 12 * n / add_ms / 1e6, "elements": n}


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_context(sample_elems: int = 1 << 25):
    """More CPU reference points on the same host: torch.optim.AdamW
    (foreach=False, the reference's "adamw" CPU path) over a 32M-element
    sample at one thread and at torch's default thread count, and the
    oracle's fp8 quantize of a bf16 activation sample (one thread)."""
    from oracle import oracle as O

    out = {}
    threads0 = torch.get_num_threads()
    try:
        for threads in sorted({1, threads0}):
            torch.set_num_threads(threads)
            p = torch.randn(sample_elems) * 0.02
            p.requires_grad_(True)
            p.grad = torch.randn(sample_elems) * 1e-4
            opt = torch.optim.AdamW([p], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, foreach=False)
            opt.step()
            t0 = time.perf_counter()
            opt.step()
            out[f"torch_adamw_params_per_s_{threads}t"] = sample_elems / (time.perf_counter() - t0)
            del opt, p
    finally:
        torch.set_num_threads(threads0)
    x = (np.random.default_rng(1).standard_normal((4096, D_MODEL)) ).astype(np.float32)
    xb = O.f32_to_bf16_bits(x).reshape(x.shape)
    rng = np.random.default_rng(2)
    p = (rng.standard_normal(sample_elems) * 0.02).astype(np.float32)
    g = O.f32_to_bf16_bits((rng.standard_normal(sample_elems) * 1e-4).astype(np.float32))
    m = np.zeros(sample_elems, np.float32)
    v = np.zeros(sample_elems, np.float32)
    cp = np.zeros(sample_elems, np.uint16)
    consts = O.host_adamw_consts(LR, BETAS, EPS, WD, 1)
    for threads in sorted({1, threads0}):
        # the oracle's C calls release the GIL: `threads` Python threads on
        # disjoint slices run on that many cores
        cuts = np.linspace(0, sample_elems, threads + 1).astype(np.int64)
        spans = list(zip(cuts[:-1], cuts[1:]))
        rows = np.linspace(0, xb.shape[0], threads + 1).astype(np.int64)
        with ThreadPoolExecutor(threads) as ex:
            t0 = time.perf_counter()
            list(ex.map(lambda s: O.adamw_host(p[s[0]:s[1]], g[s[0]:s[1]], m[s[0]:s[1]], v[s[0]:s[1]], consts, True, 1.0, cp[s[0]:s[1]]), spans))
            out[f"oracle_adamw_params_per_s_{threads}t"] = sample_elems / (time.perf_counter() - t0)
            t0 = time.perf_counter()
            qk = list(ex.map(lambda r: O.quantize(xb[r[0]:r[1]], "e4m3"), zip(rows[:-1], rows[1:])))
            out[f"oracle_fp8_quantize_GBs_{threads}t"] = xb.size * CODEC_BYTES_PER_ELEM / (time.perf_counter() - t0) / 1e9
            t0 = time.perf_counter()
            list(ex.map(lambda c: O.dequantize(c[0], c[1], "e4m3", "bf16"), qk))
            out[f"oracle_fp8_dequantize_GBs_{threads}t"] = xb.size * CODEC_BYTES_PER_ELEM / (time.perf_counter() - t0) / 1e9
    out["host_cpus"] = os.cpu_count()
    out["cpu_model"] = _cpu_model()
    out["sample"] = (f"torch AdamW and the oracle's HostAdamW (bf16 grads + bf16 copy) over {sample_elems} fp32 elements, "
                     f"oracle quantize and dequantize (-> bf16) of [4096, {D_MODEL}] bf16; threads 1 and {threads0} (torch's count)")
    return out


def read_traffic():
    """HBM bytes per AdamW launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by a plain copy's reading), if that profile is
    committed; otherwise None."""
    path = os.path.join(HERE, "profiles", "adamw_c1_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def extra_legs(device, stream):
    """The extra legs of the default run, in order: (key, what, callable)."""
    return [
        ("fold", "fold leg", lambda: bench_fold(device, stream)),
        ("release", "per-layer release leg", lambda: bench_release(device, stream)),
        ("release_host_moments", "per-layer release leg, host moments",
         lambda: bench_release(device, stream, iters=1, moments="host")),
        ("tied_fold", "tied-table row fold leg", lambda: bench_tied_fold(device, stream)),
        ("elementwise", "elementwise leg", lambda: bench_elementwise(device, stream)),
        ("c1_torch_order", "torch-order leg", lambda: bench_torch_order(device, stream)),
        ("host_moments", "host-moments leg", lambda: bench_host_moments(device)),
        ("check_host_adamw", "check_host_adamw leg (200M parameters)", lambda: bench_check_host_adamw(device)),
        ("wire", "wire leg", lambda: bench_wire(device, stream)),
        ("hbm_reference", "vendor-kernel reference leg", lambda: hbm_reference(device, stream)),
        ("configs", "configs leg (C0, C2, C3)", lambda: bench_configs(device, stream)),
        ("c1_placement", "placement leg (C1 allocated while 150 GiB are held)", lambda: bench_placement(device, stream)),
    ]


LEG_NAMES = ("fold", "release", "release_host_moments", "tied_fold", "elementwise", "c1_torch_order", "host_moments", "check_host_adamw", "wire",
             "hbm_reference", "configs", "c1_placement")


def run_legs(legs) -> dict:
    """Run (key, what, callable) legs in order; a leg that runs out of device
    memory or fails is recorded in its entry and the others go on."""
    extra = {}
    for key, what, leg in legs:
        log(what)
        try:
            extra[key] = leg()
        except torch.OutOfMemoryError as e:
            # a box with less free HBM skips the leg; the headline stands
            extra[key] = {"skipped": f"out of device memory: {str(e)[:160]}"}
        except Exception as e:  # noqa: BLE001 -- recorded in the line, the headline stands
            log(f"{what} failed: {e!r}")
            extra[key] = {"error": repr(e)[:300]}
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return extra


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)  # 0.35 s of C1 steps: the launch and sync overhead of the window is 0.1 % of it
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-codec", action="store_true", help="skip the fp8 codec leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the fused-fold, elementwise, host-moment, wire, vendor-reference and C0/C2/C3 legs")
    ap.add_argument("--codec", choices=("c1", "c4", "all"), default="all", help="activation sizes of the codec leg")
    ap.add_argument("--no-optimizer", action="store_true", help="skip the optimizer leg (profiling the other legs alone)")
    ap.add_argument("--no-configs", action="store_true", help="skip the C0/C2/C3 optimizer leg (--no-extra skips it too)")
    ap.add_argument("--leg", action="append", choices=LEG_NAMES,
                    help="run only these extra legs (repeatable), no headline, and print their JSON (for profiling one leg)")
    ap.add_argument("--c4-summary", metavar="DIR", help="summarize a rocprofv3 --kernel-trace run of --no-optimizer --codec c4 into profiles/")
    ap.add_argument("--cpu-sample", type=int, default=256 * 1024 * 1024)
    ap.add_argument("--profile-pass", action="store_true", help="launch each measured kernel a few times, untimed, for rocprofv3 --pmc runs")
    ap.add_argument("--traffic-summary", nargs="+", metavar="DIR",
                    help="summarize --pmc runs of --profile-pass into profiles/: FETCH_DIR WRITE_DIR [REQUEST_SIZE_DIR]")
    ap.add_argument("--traffic-command", default="", help="the command line recorded in the traffic summary")
    ap.add_argument("--trace-summary", nargs=2, metavar=("STEP_DIR", "CODEC_DIR"), help="summarize two rocprofv3 --kernel-trace runs into profiles/")
    ap.add_argument("--bench-json", nargs="+", metavar="OUT", help="the traced runs' own stdout (step, then codec), quoted beside the trace summary")
    args = ap.parse_args()
    if args.traffic_summary:
        if len(args.traffic_summary) not in (2, 3):
            ap.error("--traffic-summary takes FETCH_DIR WRITE_DIR [REQUEST_SIZE_DIR]")
        fd, wd = args.traffic_summary[:2]
        traffic_summary(fd, wd, args.traffic_command, args.traffic_summary[2] if len(args.traffic_summary) == 3 else None)
        return
    if args.trace_summary:
        trace_summary(*args.trace_summary, args.bench_json)
        return
    if args.c4_summary:
        c4_summary(args.c4_summary, (args.bench_json or [None])[0])
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    stream = torch.cuda.Stream(device)
    if args.profile_pass:
        with torch.cuda.stream(stream):
            profile_pass(device)
        return
    with torch.cuda.stream(stream):
        if args.leg:
            log("leg-only run: " + ", ".join(args.leg))
            print(json.dumps(run_legs([leg for leg in extra_legs(device, stream) if leg[0] in args.leg])), flush=True)
            return
        if args.no_optimizer:
            log("codec-only run")
            if args.codec in ("c1", "all"):
                print(json.dumps({"c1": bench_codec(device, stream, 8 * 2048, D_MODEL, C1_CODEC_COPIES, iters=C1_CODEC_ITERS, back_to_back=True)}), flush=True)
            if args.codec in ("c4", "all"):
                print(json.dumps({"c4": bench_c4(device, stream)}), flush=True)
            return
        log("optimizer leg")
        o = bench_optimizer(args, device, stream)
        codec = extra = None
        if not args.no_codec:
            log("codec leg")
            codec = {}
            if args.codec in ("c1", "all"):
                codec["c1_per_row"] = bench_codec(device, stream, 8 * 2048, D_MODEL, C1_CODEC_COPIES, iters=C1_CODEC_ITERS, back_to_back=True)
                torch.cuda.empty_cache()
            if args.codec in ("c4", "all"):
                codec["c4"] = bench_c4(device, stream)
                torch.cuda.empty_cache()
        if not args.no_extra:
            extra = run_legs([leg for leg in extra_legs(device, stream) if not (args.no_configs and leg[0] == "configs")])
    n = o["n_elem"]
    adam_bytes = n * ADAM_BYTES_PER_ELEM
    achieved = adam_bytes / (o["adam_ms"] * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        log("cpu baseline leg")
        # every core torch runs on: the thread count the box grants one GPU's
        # process (OMP_NUM_THREADS), which may be fewer than os.cpu_count()
        threads = torch.get_num_threads()
        rate, secs, k = cpu_baseline(args.cpu_sample, threads)
        rate1, secs1, k1 = cpu_baseline(args.cpu_sample // 4, 1, target_s=5.0)
        prate, psecs = cpu_port_baseline(args.cpu_sample // 4)
        extra = extra or {}
        extra["cpu_context"] = cpu_context()
        extra["cpu_context"]["torch_step_params_per_s_1t"] = rate1
        extra["cpu_context"]["torch_step_1t_sample"] = f"{args.cpu_sample // 4} elements, {k1} steps, {secs1:.1f} s"
        extra["cpu_context"]["oracle_port_params_per_s_1t"] = prate
        extra["cpu_context"]["oracle_port_sample"] = (f"oracle HostAdamW (C, 1 thread) over {args.cpu_sample // 4} elements, "
                                                      f"2 steps, bf16 grads + bf16 copy ({psecs:.1f} s)")
        cpu = {
            "value": rate,
            "unit": "params/s",
            "cores": threads,
            "kind": "reference",
            "sample": (f"the reference's CPU path in torch {torch.__version__}: clip_grad_norm_(foreach=False) + "
                       f"torch.optim.AdamW(foreach=False).step() + bf16 working-copy cast, {threads} threads "
                       f"(host shows {os.cpu_count()} CPUs), over a {args.cpu_sample}-element prefix of the C1 shard, "
                       f"{k} steps ({secs:.1f} s)"),
        }
    result = {
        "metric": "fused AdamW params/s & GB/s (% HBM peak); fp8 codec GB/s; 2.8B stage",
        "value": n / o["step_s"],
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": o["step_s"] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": "C1: 2.8B model, stage 1 of 2 -- 16 GPT blocks d=2560, 192 tensors, 1,258,823,680 fp32 params, bf16 grads, bf16 working copy, AdamW + global-norm clip 1.0",
            "n_params": n,
            "tensors": 192,
            "optimizer": "adamw-host op order (bit-exact), fused clip",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": read_traffic(),
        },
        "cpu_baseline": cpu,
        "kernels": {
            "adamw_ms": o["adam_ms"],
            "adamw_GBs": achieved,
            "adamw_params_per_s": n / (o["adam_ms"] * 1e-3),
            "grad_norm_ms": o["norm_ms"],
            "grad_norm_GBs": n * NORM_BYTES_PER_ELEM / (o["norm_ms"] * 1e-3) / 1e9,
            "step_GBs": n * (ADAM_BYTES_PER_ELEM + NORM_BYTES_PER_ELEM) / o["step_s"] / 1e9,
        },
        "fp8_codec": codec,
        "extra": extra,
        "grad_norm": o["grad_norm"],
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
