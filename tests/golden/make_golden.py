"""Writes the golden vectors under tests/golden/ by running the reference's own
Python (wantrain) on the CPU of the build container.

Run only where /root/reference exists (never on the GPU box):

    ATEN_CPU_CAPABILITY=avx2 MKL_ENABLE_INSTRUCTIONS=AVX2 \
        python tests/golden/make_golden.py [/root/reference]

It imports the reference for the functions that no closed form, torch
routine or invariant pins bit for bit:

* HostAdamW (runtime/optim.py:77-298): the exact fp32 parameters and moments
  after several steps, and the per-step fp32 constants `step` hands to
  _adamw_math (captured by wrapping that function), on the inputs of the
  reference's own tests/unit/test_host_adamw.py:20-28 plus a small C0-like set.
* fp8.quantize / dequantize / recover_exp (model/fp8.py:28-93) on adversarial
  rows: octave edges, extreme exponents, zero rows, NaN/Inf rows, random fp8
  code rows whose exponent recovery needs a non-zero candidate offset.
* planes.encode_scaled_fp8 / decode (codec/planes.py:85-133): the complete
  payload bytes (zlib-1 container, zstandard being absent) for the inputs of
  tests/unit/test_codecs_identity.py:59-68 and a bf16 activation.
* planes.encode / decode (codec/planes.py:141-190), the lossless byte-plane
  wire, for every wire dtype, and fp8_planes.encode / decode
  (codec/fp8_planes.py:19-52), the unscaled e4m3 nibble-plane wire, on even
  and odd element counts, plus the inputs each refuses.

The fixtures are data only (.npz, no pickles): inputs and the reference's
outputs.  The torch version they were made with is recorded in each file.
"""

from __future__ import annotations

import os
import sys
import zlib

os.environ.setdefault("ATEN_CPU_CAPABILITY", "avx2")
os.environ.setdefault("MKL_ENABLE_INSTRUCTIONS", "AVX2")

import numpy as np  # noqa: E402
import torch  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, os.path.join(REF, "src"))

from wantrain.codec import fp8_planes, planes  # noqa: E402
from wantrain.model import fp8  # noqa: E402
from wantrain.runtime import optim  # noqa: E402

torch.set_num_threads(1)
ADAMW = {"betas": (0.9, 0.95), "eps": 1e-8, "weight_decay": 0.0}  # runtime/spec.py:27
META = {"torch_version": np.array(torch.__version__), "zlib_version": np.array(zlib.ZLIB_VERSION)}


def _bits(t: torch.Tensor) -> np.ndarray:
    """A tensor's raw bits as an unsigned numpy array (bf16 -> uint16)."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return t.view(torch.uint8).numpy().copy()
    return t.numpy().copy()


# ------------------------------------------------------------------ AdamW


def _unit_params(seed=3):
    """tests/unit/test_host_adamw.py:20-23."""
    g = torch.Generator().manual_seed(seed)
    shapes = [(37, 19), (19,), (5, 3, 7), (1001,)]
    return [torch.randn(s, generator=g).requires_grad_(True) for s in shapes]


def _unit_grads(params, step, seed=5):
    """tests/unit/test_host_adamw.py:26-28."""
    g = torch.Generator().manual_seed(seed + step)
    return [torch.randn(p.shape, generator=g) * 10.0 ** (-step % 4) for p in params]


def _c0_params(seed=11):
    g = torch.Generator().manual_seed(seed)
    shapes = [(768,), (48, 96), (4099,), (3, 5)]
    return [(torch.randn(s, generator=g) * 0.02).requires_grad_(True) for s in shapes]


def _c0_grads(params, step, seed=17):
    g = torch.Generator().manual_seed(seed + step)
    return [torch.randn(p.shape, generator=g) * 1e-3 for p in params]


def _run_host_adamw(params, grads_fn, steps, lr, hp):
    captured = []
    real = optim._adamw_math

    def spy(pc, gc, m, v, c, wd):
        captured.append([c[k] for k in ("decay", "b1", "one_b1", "b2", "one_b2", "inv_bc2_sqrt", "eps", "step_size")])
        return real(pc, gc, m, v, c, wd)

    init = [p.detach().clone() for p in params]
    all_grads = []
    optim._adamw_math = spy
    try:
        opt = optim.HostAdamW(params, lr=lr, **hp)
        for step in range(steps):
            gs = grads_fn(params, step)
            all_grads.append([g.clone() for g in gs])
            for p, g in zip(params, gs):
                p.grad = g
            opt.step()
            opt.zero_grad(set_to_none=True)
    finally:
        optim._adamw_math = real
    cat = lambda ts: np.concatenate([t.detach().reshape(-1).numpy() for t in ts]).astype(np.float32)  # noqa: E731
    out = {
        "shapes": np.array([list(p.shape) + [0] * (3 - p.dim()) for p in params], dtype=np.int64),
        "numel": np.array([p.numel() for p in params], dtype=np.int64),
        "p0": cat(init),
        "grads": np.stack([cat(gs) for gs in all_grads]),
        "p": cat(params),
        "m": cat([opt.state[i]["exp_avg"] for i in range(len(params))]),
        "v": cat([opt.state[i]["exp_avg_sq"] for i in range(len(params))]),
        "consts": np.array(captured, dtype=np.float32).reshape(steps, len(params), 8),
        "hyper": np.array([lr, hp["betas"][0], hp["betas"][1], hp["eps"], hp["weight_decay"], steps], dtype=np.float64),
    }
    return out


def make_adamw():
    cases = {
        "unit": (_unit_params(), _unit_grads, 4, 1e-3, ADAMW),
        "decay": (_unit_params(), _unit_grads, 4, 1e-2, dict(ADAMW, weight_decay=0.1)),
        "c0": (_c0_params(), _c0_grads, 3, 3e-4, dict(ADAMW, weight_decay=0.1)),
    }
    arrays = dict(META)
    for name, (ps, gf, steps, lr, hp) in cases.items():
        for k, v in _run_host_adamw(ps, gf, steps, lr, hp).items():
            arrays[f"{name}_{k}"] = v
    np.savez_compressed(os.path.join(HERE, "host_adamw.npz"), **arrays)


# -------------------------------------------------------------------- fp8


def _adversarial_rows(d: int, seed: int) -> torch.Tensor:
    """float32 rows that probe fp8.py's edges; each row is one case."""
    g = torch.Generator().manual_seed(seed)
    rows = []
    for s in (-140, -133, -128, -126, -120, -100, -30, -17, -3, 0, 3, 17, 60, 100, 118, 120, 126):
        rows.append(torch.randn(d, generator=g) * 2.0**s)
    for e in (-20, -1, 0, 1, 7, 8, 9):  # amax just below, at and above an octave edge
        for f in (1 - 2.0**-9, 1.0, 1 + 2.0**-7, 1.5 - 2.0**-10, 1.9375, 1.96875):
            r = torch.randn(d, generator=g)
            r = r / r.abs().max() * 0.9
            r[d // 2] = -f * 2.0**e
            rows.append(r * 2.0**e / 2.0**e)
    z = torch.zeros(d)
    rows.append(z.clone())
    rows.append(-z)
    out = torch.randn(d, generator=g)
    out[3] = 50.0
    rows.append(out)
    tie = torch.full((d,), 1.0)
    tie[0] = 1.0625 + 2.0**-20  # near an e4m3 tie after scaling
    tie[1] = 0.96875
    rows.append(tie)
    return torch.stack(rows)


def _special_rows(d: int) -> torch.Tensor:
    rows = []
    r = torch.linspace(-3, 3, d)
    r[1] = float("nan")
    rows.append(r)
    r = torch.linspace(-3, 3, d)
    r[2] = float("inf")
    rows.append(r)
    r = torch.linspace(-3, 3, d)
    r[5] = -float("inf")
    r[6] = float("nan")
    rows.append(r)
    return torch.stack(rows)


def _fp8_code_rows(fmt: str, d: int, seed: int, n: int) -> torch.Tensor:
    """Rows drawn on the fp8 grid at random exponents: the tensors recover_exp
    is handed on the wire, some needing an offset of -1 or -2."""
    dt, _ = fp8.FORMATS[fmt]
    g = torch.Generator().manual_seed(seed)
    nan_codes = {0x7F, 0xFF} if fmt == "e4m3" else set(range(0x7C, 0x80)) | set(range(0xFC, 0x100))
    ok = torch.tensor([c for c in range(256) if c not in nan_codes], dtype=torch.int64)
    rows = []
    for i in range(n):
        mode = i % 4
        if mode == 0:
            codes = ok[torch.randint(len(ok), (d,), generator=g)]
        elif mode == 1:  # large and tiny magnitudes together
            codes = ok[torch.randint(len(ok), (d,), generator=g)]
            codes[0] = 0x7E if fmt == "e4m3" else 0x7B
            codes[1] = 0x01
        elif mode == 2:  # only small codes
            codes = torch.randint(0, 24, (d,), generator=g)
        else:
            codes = ok[torch.randint(len(ok), (d,), generator=g)]
            codes[d - 1] = 0x78 if fmt == "e4m3" else 0x78
        q = codes.to(torch.uint8).view(dt)
        k = int(torch.randint(-40, 40, (1,), generator=g))
        rows.append(q.to(torch.float32) * 2.0**k)
    return torch.stack(rows)


def _recover_rows(t: torch.Tensor, fmt: str):
    """recover_exp row by row: a row with no exact k raises for its whole
    tensor, so each row is its own [1, d] call.  -> (k, ok) per row."""
    rec, okrow = [], []
    for r in t:
        try:
            rec.append(int(fp8.recover_exp(r.reshape(1, -1), fmt)))
            okrow.append(1)
        except ValueError:
            rec.append(0)
            okrow.append(0)
    return np.array(rec, dtype=np.int32), np.array(okrow, dtype=np.int8)


def make_fp8():
    arrays = dict(META)
    d = 32
    base = _adversarial_rows(d, 7)
    special = _special_rows(d)
    for fmt in ("e4m3", "e5m2"):
        for dname, dtype in (("f32", torch.float32), ("bf16", torch.bfloat16)):
            pre = f"{fmt}_{dname}"
            x = base.to(dtype)
            arrays[f"{pre}_x"] = _bits(x)
            arrays[f"{pre}_k"] = fp8.scale_exp(x, fmt).reshape(-1).numpy()
            q, k = fp8.quantize(x, fmt)
            arrays[f"{pre}_q"] = _bits(q)
            arrays[f"{pre}_qk"] = k.reshape(-1).numpy()
            arrays[f"{pre}_deq_f32"] = _bits(fp8.dequantize(q, k))
            rt = fp8.roundtrip(x, fmt)
            arrays[f"{pre}_rt"] = _bits(rt)
            rec, okrow = _recover_rows(rt, fmt)
            arrays[f"{pre}_rec"] = rec
            arrays[f"{pre}_rec_ok"] = okrow
            xs = special.to(dtype)
            arrays[f"{pre}_sx"] = _bits(xs)
            qs, ks = fp8.quantize(xs, fmt)
            arrays[f"{pre}_sq"] = _bits(qs)
            arrays[f"{pre}_sk"] = ks.reshape(-1).numpy()
            arrays[f"{pre}_sdeq"] = _bits(fp8.dequantize(qs, ks, dtype))
            # recover_exp row by row (a row with no exact k raises for its tensor)
            codes = _fp8_code_rows(fmt, d, 99 if fmt == "e4m3" else 98, 96).to(dtype)
            perturbed = codes.clone()
            perturbed[::7, 4] = perturbed[::7, 4] * (1 + 2.0**-6)  # off the grid: no k fits
            cand = torch.cat([codes, perturbed[::7]])
            rec, okrow = _recover_rows(cand, fmt)
            arrays[f"{pre}_cand"] = _bits(cand)
            arrays[f"{pre}_cand_k"] = rec
            arrays[f"{pre}_cand_ok"] = okrow
    np.savez_compressed(os.path.join(HERE, "fp8_rows.npz"), **arrays)


# ------------------------------------------------------------------- wire


def make_wire():
    arrays = dict(META)
    cases = []
    x = torch.randn(3, 8, 32) * 1e-4  # tests/unit/test_codecs_identity.py:62
    for fmt in ("e4m3", "e5m2"):
        cases.append((f"unit_{fmt}", fp8.roundtrip(x, fmt), fmt))
    g = torch.Generator().manual_seed(21)
    act = torch.randn(2, 16, 64, generator=g).to(torch.bfloat16)
    act[0, 3, 5] = 50.0
    for fmt in ("e4m3", "e5m2"):
        cases.append((f"act_{fmt}", fp8.roundtrip(act, fmt), fmt))
    vec = fp8.roundtrip(torch.randn(1, 100, generator=g) * 3, "e4m3").reshape(100)
    cases.append(("vec_e4m3", vec, "e4m3"))
    for name, t, fmt in cases:
        payload, shape = planes.encode_scaled_fp8(t, fmt)
        arrays[f"{name}_t"] = _bits(t)
        arrays[f"{name}_dtype"] = np.array(str(t.dtype))
        arrays[f"{name}_shape"] = np.array(shape, dtype=np.int64)
        arrays[f"{name}_payload"] = np.frombuffer(payload, dtype=np.uint8).copy()
        arrays[f"{name}_decoded"] = _bits(planes.decode(payload, shape))
    arrays["names"] = np.array([c[0] for c in cases])
    np.savez_compressed(os.path.join(HERE, "wire.npz"), **arrays)


# ----------------------------------------------------------- plane codecs


def _plane_inputs():
    """One small tensor per wire dtype (codec/planes.py:63-70), with the
    values a byte split must carry: signs, zeros, NaN/Inf, extremes."""
    g = torch.Generator().manual_seed(41)
    x = torch.randn(3, 7, 33, generator=g) * 4
    x.view(-1)[:6] = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 1e-40])
    out = [
        ("f32", x.clone()),
        ("bf16", x.to(torch.bfloat16)),
        ("f16", (x / 8).to(torch.float16)),
        ("e4m3", (x / 8).clamp(-400, 400).to(torch.float8_e4m3fn)),
        ("e5m2", (x / 8).to(torch.float8_e5m2)),
        ("i64", torch.randint(-(1 << 62), 1 << 62, (5, 13), generator=g, dtype=torch.int64)),
        ("bf16_one", torch.tensor([1.5], dtype=torch.bfloat16)),
    ]
    return out


def _fp8_plane_inputs():
    """e4m3-representable tensors (the fp8_planes precondition), even and
    odd element counts, fp32 and bf16."""
    g = torch.Generator().manual_seed(43)
    codes = torch.randint(0, 256, (4, 9, 27), generator=g, dtype=torch.int64)
    codes[(codes & 0x7F) == 0x7F] = 0x11  # no NaN codes
    q = codes.to(torch.uint8).view(torch.float8_e4m3fn)
    return [
        ("odd_f32", q.to(torch.float32)),
        ("odd_bf16", q.to(torch.bfloat16)),
        ("even_f32", q.to(torch.float32).reshape(-1)[:512].reshape(16, 32)),
        ("one_f32", q.to(torch.float32).reshape(-1)[:1]),
    ]


def make_planes():
    arrays = dict(META)
    names = []
    for name, t in _plane_inputs():
        payload, shape = planes.encode(t)
        arrays[f"p_{name}_t"] = np.frombuffer(t.contiguous().view(torch.uint8).numpy().tobytes(), dtype=np.uint8).copy()
        arrays[f"p_{name}_dtype"] = np.array(str(t.dtype))
        arrays[f"p_{name}_shape"] = np.array(shape, dtype=np.int64)
        arrays[f"p_{name}_payload"] = np.frombuffer(payload, dtype=np.uint8).copy()
        back = planes.decode(payload, shape)
        arrays[f"p_{name}_decoded"] = np.frombuffer(back.contiguous().view(torch.uint8).numpy().tobytes(), dtype=np.uint8).copy()
        names.append(name)
    arrays["plane_names"] = np.array(names)
    names = []
    for name, t in _fp8_plane_inputs():
        payload, shape = fp8_planes.encode(t)
        arrays[f"n_{name}_t"] = _bits(t)
        arrays[f"n_{name}_dtype"] = np.array(str(t.dtype))
        arrays[f"n_{name}_shape"] = np.array(shape, dtype=np.int64)
        arrays[f"n_{name}_payload"] = np.frombuffer(payload, dtype=np.uint8).copy()
        arrays[f"n_{name}_decoded"] = _bits(fp8_planes.decode(payload, shape))
        names.append(name)
    arrays["nibble_names"] = np.array(names)
    # inputs fp8_planes.encode refuses (not e4m3-representable), one per row
    bad = torch.tensor([[1.0, 2.0, 3.0, 1.0 + 2.0**-5], [0.0, float("nan"), 1.0, 2.0], [500.0, 1.0, 2.0, 3.0], [2.0**-10, 0, 0, 0]])
    refused = []
    for r in bad:
        try:
            fp8_planes.encode(r)
            refused.append(0)
        except AssertionError:
            refused.append(1)
    arrays["n_bad_t"] = _bits(bad)
    arrays["n_bad_refused"] = np.array(refused, dtype=np.int8)
    np.savez_compressed(os.path.join(HERE, "planes.npz"), **arrays)


if __name__ == "__main__":
    which = sys.argv[2:] or ["adamw", "fp8", "wire", "planes"]
    for w in which:
        {"adamw": make_adamw, "fp8": make_fp8, "wire": make_wire, "planes": make_planes}[w]()
    print("golden vectors written to", HERE, which)
