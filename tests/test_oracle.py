"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is independent of the oracle's own formulation:
* torch's own conversions (`.to(float8_*)`, `.to(bfloat16)`) exhaustively or
  on large samples -- torch is the library the reference calls for them;
* golden vectors the reference itself produced (tests/golden/make_golden.py);
* closed forms: frexp by Python's math.frexp, exact rational sums, the first
  Adam step moving every parameter by lr * sign(g);
* torch's clip_grad_norm_ and AdamW run as black boxes.
Mutation checks at the end show that a plausible mistake fails a golden test.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from conftest import golden

FP8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------- conversions


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_fp8_encode_equals_torch_on_every_bf16_pattern(oracle, fmt):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = oracle.bf16_bits_to_f32(h)
    mine = oracle.fp8_encode(f, fmt)
    ref = torch.from_numpy(f.copy()).to(FP8[fmt]).view(torch.uint8).numpy()
    assert np.array_equal(mine, ref)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_fp8_encode_equals_torch_on_fp32_patterns(oracle, fmt):
    # every 4099th fp32 pattern (~1M values: both signs, subnormals, NaN
    # payloads) plus the rounding edges of both formats
    u = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)
    edges = np.array(
        [448, 464, 464.0001, 479.99, 480, 57344, 61439.99, 61440, 65535.9, 65536, 2.0**-9, 2.0**-10, 2.0**-10 * 1.0001,
         2.0**-16, 2.0**-17, 2.0**-17 * 1.0001, 3 * 2.0**-11, 1.0625, 1.1875, 0.0, float("inf"), float("nan")],
        dtype=np.float32,
    )
    x = np.concatenate([u.view(np.float32), edges, -edges])
    mine = oracle.fp8_encode(x, fmt)
    ref = torch.from_numpy(x.copy()).to(FP8[fmt]).view(torch.uint8).numpy()
    assert np.array_equal(mine, ref)


def test_fp8_decode_tables_closed_form_and_torch(oracle):
    e4 = oracle.fp8_decode_table("e4m3")
    e5 = oracle.fp8_decode_table("e5m2")
    # the formats' definitions: largest finite, smallest subnormal, smallest normal, NaN/Inf codes
    assert e4[0x7E] == 448.0 and e4[0x01] == 2.0**-9 and e4[0x08] == 2.0**-6 and np.isnan(e4[0x7F]) and np.isnan(e4[0xFF])
    assert e5[0x7B] == 57344.0 and e5[0x01] == 2.0**-16 and e5[0x04] == 2.0**-14 and np.isinf(e5[0x7C])
    assert all(np.isnan(e5[c]) for c in (0x7D, 0x7E, 0x7F, 0xFD, 0xFE, 0xFF))
    assert np.signbit(e4[0x80]) and e4[0x80] == 0.0
    pos4 = e4[:0x7F]
    assert np.all(np.diff(pos4) > 0)  # codes are ordered by value
    for fmt, tab in (("e4m3", e4), ("e5m2", e5)):
        ref = torch.arange(256, dtype=torch.uint8).view(FP8[fmt]).float().numpy()
        assert np.array_equal(np.isnan(tab), np.isnan(ref))
        ok = ~np.isnan(ref)
        assert np.array_equal(tab[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_bf16_rounding_equals_torch(oracle):
    """Non-NaN values: bit for bit torch's CPU cast.  NaN: c10's scalar rule
    0x7FC0 (BFloat16.h:100-114), which torch's GPU kernels use; torch's AVX2
    CPU cast writes 0xFFFF instead, so there only NaN-ness is compared (the GPU
    tests hold the kernels to torch-on-GPU bits, NaN included)."""
    rng = np.random.default_rng(0)
    u = rng.integers(0, 1 << 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 1 << 16, size=10000, dtype=np.uint32) << 16) | 0x8000
    x = np.concatenate([u, ties, np.array([0x7FC00001, 0xFFC00000, 0x7F800000, 0x7F7FFFFF, 0x00008000], dtype=np.uint32)]).view(np.float32)
    mine = oracle.f32_to_bf16_bits(x)
    ref = _bf16_bits(torch.from_numpy(x.copy()).to(torch.bfloat16))
    nan = np.isnan(x)
    assert np.array_equal(mine[~nan], ref[~nan])
    assert np.all(mine[nan] == 0x7FC0)
    assert np.all(np.isnan(oracle.bf16_bits_to_f32(ref[nan])))
    # the scalar c10 path (one element at a time) agrees with the oracle on NaN too
    for bits in (0x7FC00001, 0xFFC00000, 0x7F800001):
        one = torch.tensor([np.uint32(bits).view(np.float32)], dtype=torch.float32)
        assert oracle.f32_to_bf16_bits(one.numpy())[0] == 0x7FC0


# ---------------------------------------------------------------- scale_exp


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_scale_exp_is_frexp_of_the_row_max(oracle, fmt):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 33)) * np.exp2(rng.integers(-60, 60, size=(64, 1)))).astype(np.float32)
    x[5] = 0.0
    k = oracle.scale_exp(x, fmt)
    eb = oracle.EBIAS[fmt]
    for r in range(x.shape[0]):
        amax = float(np.max(np.abs(x[r])))
        want = 0 if amax == 0 else math.frexp(amax)[1] - eb
        assert k[r] == want
        if amax:
            s = amax * 2.0 ** -int(k[r])
            assert 2.0 ** (eb - 1) <= s < 2.0**eb  # the scaled row max sits in the top octave


# ------------------------------------------------------------- golden fp8

_G8 = [(f, d) for f in ("e4m3", "e5m2") for d in ("f32", "bf16")]


def _x(arr, dname):
    return arr.astype(np.float32) if dname == "f32" else arr.astype(np.uint16)


def _nan_code(q: np.ndarray, fmt: str) -> np.ndarray:
    low = q & 0x7F
    return low == 0x7F if fmt == "e4m3" else low > 0x7C


def _same_codes(a: np.ndarray, b: np.ndarray, fmt: str) -> bool:
    """Equal fp8 codes, except that a NaN's sign is not compared: a NaN made
    inside the arithmetic (0 * Inf when 2^-k overflows the dtype) takes the
    device's default NaN, negative on x86 (where the golden vectors were made)
    and positive on AMD GPUs (which the oracle and the kernels follow)."""
    na, nb = _nan_code(a, fmt), _nan_code(b, fmt)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb]))


def _same_bf16(a: np.ndarray, b: np.ndarray) -> bool:
    """Equal bf16 bits, NaN compared as NaN (x86's AVX2 cast writes 0xFFFF)."""
    fa = (a.astype(np.uint32) << 16).view(np.float32)
    fb = (b.astype(np.uint32) << 16).view(np.float32)
    na, nb = np.isnan(fa), np.isnan(fb)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb]))


@pytest.mark.parametrize("fmt,dname", _G8)
def test_quantize_dequantize_match_reference_golden(oracle, fmt, dname):
    g = golden("fp8_rows.npz")
    pre = f"{fmt}_{dname}"
    x = _x(g[f"{pre}_x"], dname)
    assert np.array_equal(oracle.scale_exp(x, fmt), g[f"{pre}_k"])
    q, k = oracle.quantize(x, fmt)
    assert _same_codes(q, g[f"{pre}_q"], fmt) and np.array_equal(k, g[f"{pre}_qk"])
    deq = oracle.dequantize(q, k, fmt, "f32")
    ref = g[f"{pre}_deq_f32"]
    assert np.array_equal(np.isnan(deq), np.isnan(ref))
    assert np.array_equal(deq[~np.isnan(deq)].view(np.uint32), ref[~np.isnan(ref)].view(np.uint32))
    rt = oracle.roundtrip(x, fmt)
    rref = g[f"{pre}_rt"]
    if dname == "f32":
        assert np.array_equal(np.isnan(rt), np.isnan(rref))
        assert np.array_equal(rt[~np.isnan(rt)].view(np.uint32), rref[~np.isnan(rref)].view(np.uint32))
    else:
        assert _same_bf16(rt, rref)


@pytest.mark.parametrize("fmt,dname", _G8)
def test_special_rows_match_reference_golden(oracle, fmt, dname):
    g = golden("fp8_rows.npz")
    pre = f"{fmt}_{dname}"
    x = _x(g[f"{pre}_sx"], dname)
    q, k = oracle.quantize(x, fmt)
    assert _same_codes(q, g[f"{pre}_sq"], fmt) and np.array_equal(k, g[f"{pre}_sk"])
    out = oracle.dequantize(q, k, fmt, "f32" if dname == "f32" else "bf16")
    ref = g[f"{pre}_sdeq"]
    if dname == "bf16":
        assert _same_bf16(out, ref)
    else:
        assert np.array_equal(np.isnan(out), np.isnan(ref))
        assert np.array_equal(out[~np.isnan(out)], ref[~np.isnan(ref)])


@pytest.mark.parametrize("fmt,dname", _G8)
def test_recover_exp_matches_reference_golden(oracle, fmt, dname):
    g = golden("fp8_rows.npz")
    pre = f"{fmt}_{dname}"
    for src, kk, ok in (("rt", "rec", "rec_ok"), ("cand", "cand_k", "cand_ok")):
        t = _x(g[f"{pre}_{src}"], dname)
        want_k, want_ok = g[f"{pre}_{kk}"], g[f"{pre}_{ok}"]
        for r in range(t.shape[0]):
            k, bad = oracle.recover_exp(t[r : r + 1], fmt)
            assert (bad == 0) == bool(want_ok[r]), (src, r)
            if want_ok[r]:
                assert k[0] == want_k[r], (src, r)


def test_golden_recover_rows_exercise_every_branch():
    """The golden candidate rows are adversarial: some need an offset other
    than 0 and some have no exact exponent at all."""
    g = golden("fp8_rows.npz")
    offsets, failures = set(), 0
    for fmt in ("e4m3", "e5m2"):
        for dname in ("f32", "bf16"):
            pre = f"{fmt}_{dname}"
            t = g[f"{pre}_cand"].astype(np.float32) if dname == "f32" else (g[f"{pre}_cand"].astype(np.uint32) << 16).view(np.float32)
            for r in range(t.shape[0]):
                if not g[f"{pre}_cand_ok"][r]:
                    failures += 1
                    continue
                amax = float(np.max(np.abs(t[r])))
                base = math.frexp(amax)[1] - (8 if fmt == "e4m3" else 15) if amax else 0
                offsets.add(int(g[f"{pre}_cand_k"][r]) - base)
    assert failures > 0 and offsets - {0}, offsets


# ------------------------------------------------------------- golden AdamW


@pytest.mark.parametrize("case", ["unit", "decay", "c0"])
def test_host_adamw_matches_reference_golden(oracle, case):
    g = golden("host_adamw.npz")
    lr, b1, b2, eps, wd, steps = g[f"{case}_hyper"]
    steps = int(steps)
    numel = g[f"{case}_numel"]
    p = g[f"{case}_p0"].copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for step in range(steps):
        c = oracle.host_adamw_consts(lr, (b1, b2), eps, wd, step + 1)
        assert np.array_equal(c, g[f"{case}_consts"][step][0])  # every tensor shares the step's constants
        assert all(np.array_equal(c, row) for row in g[f"{case}_consts"][step])
        oracle.adamw_host(p, g[f"{case}_grads"][step].copy(), m, v, c, wd != 0)
    assert sum(numel) == p.size
    assert np.array_equal(p.view(np.uint32), g[f"{case}_p"].view(np.uint32))
    assert np.array_equal(m.view(np.uint32), g[f"{case}_m"].view(np.uint32))
    assert np.array_equal(v.view(np.uint32), g[f"{case}_v"].view(np.uint32))


def test_host_adamw_first_step_moves_by_lr_sign_g(oracle):
    """t = 1 from zero moments: m = (1-b1) g, v = (1-b2) g^2, and with the
    bias corrections the update is lr * g / (|g| + eps') -> lr * sign(g)."""
    rng = np.random.default_rng(2)
    p0 = np.zeros(10000, dtype=np.float32)  # p = -update exactly: no cancellation in the check
    g = (rng.standard_normal(10000) * 0.1).astype(np.float32)
    g[np.abs(g) < 1e-3] = 1e-3
    lr = 1e-3
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    oracle.adamw_host(p, g, m, v, oracle.host_adamw_consts(lr, (0.9, 0.95), 1e-8, 0.0, 1), False)
    np.testing.assert_allclose(-p, lr * np.sign(g), rtol=2e-5, atol=0)
    np.testing.assert_allclose(m, 0.1 * g, rtol=1e-6)
    np.testing.assert_allclose(v, 0.05 * g.astype(np.float64) ** 2, rtol=1e-6)


@pytest.mark.parametrize("foreach", [False, True])
def test_torch_order_oracle_is_adamw(oracle, foreach):
    """The restatement of torch's GPU (foreach) op order against
    torch.optim.AdamW itself on the CPU, at the bounds measured there: the
    CPU kernels round some ops differently (addcmul as (value * t1) * t2
    where the GPU fuses value * (t1 * t2) into the add; the update's
    addcdiv likewise), so exp_avg is bit-identical, exp_avg_sq within 4 ulp,
    and the parameters within the reference's own tolerance for 'it is
    AdamW' (test_host_adamw.py:70-77).  The GPU kernel itself is held to
    torch's GPU AdamW bit for bit (0 ulp) on parameters and both moments
    (tests/test_gpu_adamw.py); the north star's contract for it is 1 ulp."""
    from gpu_util import ulp_distance

    rng = np.random.default_rng(3)
    p0 = rng.standard_normal(50000).astype(np.float32)
    tp = torch.from_numpy(p0.copy()).requires_grad_(True)
    opt = torch.optim.AdamW([tp], lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=foreach)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for step in range(5):
        gr = (rng.standard_normal(50000) * 10.0 ** (-step % 4)).astype(np.float32)
        tp.grad = torch.from_numpy(gr.copy())
        opt.step()
        oracle.adamw_torch(p, gr, m, v, oracle.torch_adamw_consts(1e-2, (0.9, 0.95), 1e-8, 0.1, step + 1), True)
    np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-5, atol=1e-6)
    assert int(ulp_distance(m, opt.state[tp]["exp_avg"].numpy()).max()) == 0
    assert int(ulp_distance(v, opt.state[tp]["exp_avg_sq"].numpy()).max()) <= 4


def test_bf16_grads_equal_their_fp32_widening(oracle):
    """bf16 grads enter as their exact fp32 widening (pieces.fold_start)."""
    rng = np.random.default_rng(4)
    gb = oracle.f32_to_bf16_bits(rng.standard_normal(3001).astype(np.float32))
    gf = oracle.bf16_bits_to_f32(gb)
    c = oracle.host_adamw_consts(3e-4, (0.9, 0.95), 1e-8, 0.1, 1)
    a = [rng.standard_normal(3001).astype(np.float32) for _ in range(3)]
    a[2] = np.abs(a[2]) * 1e-4  # a second moment is non-negative
    b = [x.copy() for x in a]
    oracle.adamw_host(a[0], gb, a[1], a[2], c, True)
    oracle.adamw_host(b[0], gf, b[1], b[2], c, True)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


# ------------------------------------------------------------- golden wire


def test_wire_image_matches_reference_golden(oracle):
    g = golden("wire.npz")
    for name in g["names"]:
        name = str(name)
        dt = str(g[f"{name}_dtype"])
        t = g[f"{name}_t"]
        t = t.astype(np.uint16) if "bfloat16" in dt else t.astype(np.float32)
        payload = oracle.wire_encode(t.reshape(tuple(g[f"{name}_shape"])), "e5m2" if name.endswith("e5m2") else "e4m3")
        assert payload == g[f"{name}_payload"].tobytes(), name
        out = oracle.wire_decode(payload, tuple(g[f"{name}_shape"]))
        assert np.array_equal(out.view(np.uint32), g[f"{name}_decoded"].view(np.uint32)), name


def test_wire_refuses_an_unnarrowed_tensor(oracle):
    x = (np.random.default_rng(5).standard_normal((3, 8, 32)) * 1e-4).astype(np.float32)
    with pytest.raises(ValueError, match="recipe mismatch"):
        oracle.wire_encode(x, "e4m3")


# -------------------------------------------------------- norm and clipping


def test_sumsq_equals_exact_rational_sum(oracle):
    rng = np.random.default_rng(6)
    gs = [(rng.standard_normal(n) * 10.0 ** rng.integers(-6, 3)).astype(np.float32) for n in (1, 17, 1000, 4097)]
    gs.append(oracle.f32_to_bf16_bits(rng.standard_normal(999).astype(np.float32)))
    exact = Fraction(0)
    for g in gs:
        vals = g if g.dtype == np.float32 else oracle.bf16_bits_to_f32(g)
        exact += sum(Fraction(float(x)) ** 2 for x in vals)
    got = oracle.sumsq(gs)
    assert abs(Fraction(got) - exact) <= exact * Fraction(1, 10**14)


def test_clip_coefficient_equals_torch_clip_grad_norm(oracle):
    """For every max_norm torch's formula covers: 0 zeroes the gradients, a
    negative one flips them (the clamp is max=1 only)."""
    rng = np.random.default_rng(7)
    for max_norm in (1.0, 0.5, 0.0, -2.0):
        for scale in (1e-3, 0.3, 10.0, 1e3):
            ps = []
            for n in (100, 1, 333):
                p = torch.zeros(n, requires_grad=True)
                g = torch.from_numpy((rng.standard_normal(n) * scale).astype(np.float32))
                g[0] = 1.0  # after clipping this element is the coefficient itself
                p.grad = g
                ps.append(p)
            total = torch.nn.utils.clip_grad_norm_(ps, max_norm=max_norm, foreach=False)
            coef_torch = float(ps[0].grad[0])
            assert np.float32(oracle.clip_coef(float(total), max_norm)) == np.float32(coef_torch), (max_norm, scale)


# ---------------------------------------------------------------- mutations


def test_a_swapped_constant_fails_the_adamw_golden(oracle):
    """WOULD-FAIL-IF check: exchanging b1 and 1-b1 is caught."""
    g = golden("host_adamw.npz")
    p = g["unit_p0"].copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    for step in range(4):
        c = oracle.host_adamw_consts(1e-3, (0.9, 0.95), 1e-8, 0.0, step + 1)
        c[1], c[2] = c[2], c[1]
        oracle.adamw_host(p, g["unit_grads"][step].copy(), m, v, c, False)
    assert not np.array_equal(p, g["unit_p"])


def test_a_wrong_format_bias_fails_the_fp8_golden(oracle):
    """WOULD-FAIL-IF check: quantizing e4m3 rows with e5m2's bias is caught."""
    g = golden("fp8_rows.npz")
    x = g["e4m3_f32_x"].astype(np.float32)
    k = oracle.scale_exp(x, "e5m2")
    assert not np.array_equal(k, g["e4m3_f32_k"])
    q, _ = oracle.quantize(x, "e5m2")
    assert not np.array_equal(q, g["e4m3_f32_q"])


# ----------------------------------------------------------- plane codecs


def test_byte_plane_payloads_match_reference_golden(oracle):
    """codec/planes.py:141-190: the oracle's payload equals the reference's,
    byte for byte, for every wire dtype; decoding restores the bytes."""
    g = golden("planes.npz")
    for name in g["plane_names"]:
        name = str(name)
        raw = g[f"p_{name}_t"]
        dname = str(g[f"p_{name}_dtype"]).replace("torch.", "")
        payload = oracle.planes_encode(raw, dname)
        assert payload == g[f"p_{name}_payload"].tobytes(), name
        did, back = oracle.planes_decode(payload)
        assert did == oracle.PLANE_IDS[dname] and np.array_equal(back, g[f"p_{name}_decoded"]), name


def test_byte_planes_are_the_textbook_split(oracle):
    """Plane j of a 4-byte little-endian element is byte 3 - j: the same as
    numpy's big-endian view of the elements, read column by column."""
    x = np.random.default_rng(0).integers(0, 2**32, 1001, dtype=np.uint64).astype(np.uint32)
    planes = oracle.byte_planes(x.view(np.uint8), 4)
    be = x.astype(">u4").view(np.uint8).reshape(-1, 4)
    for j in range(4):
        assert np.array_equal(planes[j], be[:, j])


def test_f32_planes_are_the_transposed_little_endian_bytes(oracle):
    """codec/f32_planes.py:17-33: the decompressed body is the elements'
    little-endian bytes read column by column (numpy's transpose of the
    (n, 4) byte matrix: byte 0 of every element first), behind an <Q>
    count; decode inverts it for every bit pattern, including NaN payloads,
    infinities, -0.0 and subnormals, and for no elements at all."""
    import struct
    import zlib

    rng = np.random.default_rng(3)
    for n in (0, 1, 7, 1001):
        x = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        x[: min(n, 5)] = np.array([0x7FC00001, 0xFF800000, 0x80000000, 0x00000001, 0x7F7FFFFF], dtype=np.uint32)[: min(n, 5)]
        raw = x.view(np.uint8)
        payload = oracle.f32_planes_encode(raw)
        assert struct.unpack_from("<Q", payload, 0) == (n,)
        body = np.frombuffer(zlib.decompress(payload[8:]), dtype=np.uint8)
        assert np.array_equal(body, raw.reshape(-1, 4).T.reshape(-1))
        assert np.array_equal(oracle.f32_planes_decode(payload), raw)


def test_nibble_payloads_match_reference_golden(oracle):
    """codec/fp8_planes.py:19-52: payload bytes and decoded values equal the
    reference's; the inputs it refuses are refused."""
    g = golden("planes.npz")
    for name in g["nibble_names"]:
        name = str(name)
        t = g[f"n_{name}_t"]
        payload = oracle.fp8_planes_encode(t)
        assert payload == g[f"n_{name}_payload"].tobytes(), name
        assert np.array_equal(oracle.fp8_planes_decode(payload).view(np.uint32), g[f"n_{name}_decoded"].reshape(-1).view(np.uint32))
    for row, refused in zip(g["n_bad_t"], g["n_bad_refused"]):
        if refused:
            with pytest.raises(AssertionError):
                oracle.fp8_planes_encode(row)


def test_nibble_packing_is_numpys_packbits(oracle):
    """fp8_planes.py:27-30 packs 4-bit values with np.packbits: the oracle's
    nibble arithmetic equals that library routine on odd and even counts."""
    rng = np.random.default_rng(1)
    for n in (1, 2, 7, 1000, 1001):
        c = rng.integers(0, 256, n, dtype=np.uint8)
        hi, lo = oracle.nibble_planes(c)
        for plane, nib in ((hi, c >> 4), (lo, c & 0x0F)):
            ref = np.packbits(np.unpackbits(nib.reshape(-1, 1), axis=1, count=8)[:, 4:])
            assert np.array_equal(plane, ref)


@pytest.mark.parametrize("gdt", ["bf16", "f32"])
def test_fold_add_bf16_equals_torch_add_on_a_bf16_sum(oracle, gdt):
    """OrderedAccumulator's fold into a bf16 sum is torch's in-place add on a
    bf16 tensor (runtime/accumulate.py:101-102): bit for bit torch's CPU
    add_, over random bf16 sums (every exponent, subnormals, +-0, +-Inf)
    and bf16 or fp32 parts; NaN results compared as NaN (torch's AVX2 cast
    writes another NaN pattern than c10's 0x7FC0, which the oracle and the
    GPU use)."""
    rng = np.random.default_rng(7 if gdt == "bf16" else 8)
    n = 400_000
    acc = rng.integers(0, 1 << 16, size=n, dtype=np.uint32).astype(np.uint16)
    acc[:6] = [0x0000, 0x8000, 0x7F80, 0xFF80, 0x0001, 0x8001]
    if gdt == "bf16":
        g = rng.integers(0, 1 << 16, size=n, dtype=np.uint32).astype(np.uint16)
        g[:6] = [0x8000, 0x0000, 0xFF80, 0x7F80, 0x8001, 0x0001]
        g_t = torch.from_numpy(g.view(np.int16).copy()).view(torch.bfloat16)
    else:
        g = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32).view(np.float32)
        g_t = torch.from_numpy(g.copy())
    acc_t = torch.from_numpy(acc.view(np.int16).copy()).view(torch.bfloat16)
    acc_t.add_(g_t)
    want = acc_t.view(torch.int16).numpy().view(np.uint16)
    mine = acc.copy()
    oracle.fold_add_bf16(mine, g)
    nan = np.isnan(oracle.bf16_bits_to_f32(want))
    assert np.array_equal(mine[~nan], want[~nan])
    assert np.all(mine[nan] == 0x7FC0)
    # a planted mistake: the add rounded straight from the two bf16 values
    # in bf16 (no fp32 step) would differ from torch somewhere
    if gdt == "f32":
        with np.errstate(over="ignore", invalid="ignore"):
            wrong = oracle.f32_to_bf16_bits(oracle.bf16_bits_to_f32(acc) + oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(g)))
        assert not np.array_equal(wrong[~nan], want[~nan])
