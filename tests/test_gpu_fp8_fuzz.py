"""Property-based fuzz of the fp8 codec on the GPU against the oracle:
random row counts and lengths (every register path, the block-row and the
split paths, odd lengths), bf16 or fp32 input, e4m3 or e5m2, per-row or
per-tensor, rows at exponents across the whole range (the instruction path
and the restatement path), with NaN, +-Inf, +-0 and subnormals sprinkled
in.  quantize (codes and k), dequantize, the fused round trip and
recover_exp on the round trip must equal the oracle's (model/fp8.py:28-93);
a NaN made inside the arithmetic is compared as a NaN code.  Derandomized."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from gpu_util import bits, say

pytestmark = pytest.mark.gpu

FUZZ = settings(max_examples=80, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
COLS = [1, 3, 7, 8, 16, 24, 100, 512, 768, 1000, 2560, 3072, 3200, 4096, 4104, 8192, 8200, 16408]


def _nan_codes(q: np.ndarray, fmt: str) -> np.ndarray:
    return ((q & 0x7F) == 0x7F) if fmt == "e4m3" else ((q & 0x7F) > 0x7C)


def _codes_equal(a: np.ndarray, b: np.ndarray, fmt: str) -> bool:
    na, nb = _nan_codes(a, fmt), _nan_codes(b, fmt)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb]))


def _vals_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit patterns equal (bf16 as uint16, fp32 as float32), any NaN equal to any NaN."""
    if a.dtype == np.uint16:
        na, nb = (a & 0x7FFF) > 0x7F80, (b & 0x7FFF) > 0x7F80
        return bool(np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb]))
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


@FUZZ
@given(
    rows=st.integers(1, 24),
    cols=st.sampled_from(COLS),
    bf16=st.booleans(),
    fmt=st.sampled_from(["e4m3", "e5m2"]),
    per_tensor=st.booleans(),
    specials=st.sampled_from([0.0, 0.0, 1e-3, 0.05]),
    seed=st.integers(0, 2**16),
)
def test_codec_matches_the_oracle(oracle, rows, cols, bf16, fmt, per_tensor, specials, seed):
    from elysium_wan_amd import fp8

    rng = np.random.default_rng(seed)
    e = rng.integers(-135, 125, size=(rows, 1))
    x = (rng.standard_normal((rows, cols)) * np.exp2(e.astype(np.float64))).astype(np.float32)
    if specials:
        pick = rng.random((rows, cols)) < specials
        pool = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -3e-39, 1e-45], dtype=np.float32)
        x[pick] = pool[rng.integers(0, pool.size, size=int(pick.sum()))]
    if bf16:
        xb = oracle.f32_to_bf16_bits(x).reshape(x.shape)
        xt = torch.from_numpy(xb.view(np.int16).copy()).view(torch.bfloat16).cuda()
        host = xb
    else:
        xt = torch.from_numpy(x.copy()).cuda()
        host = x
    say("fp8 fuzz", rows, cols, "bf16" if bf16 else "f32", fmt, "tensor" if per_tensor else "row", specials, seed)
    ohost = host.reshape(1, -1) if per_tensor else host
    oq, ok = oracle.quantize(ohost, fmt)
    q, k = fp8.quantize(xt, fmt, per_tensor=per_tensor)
    qb = bits(q).reshape(-1)
    assert _codes_equal(qb, oq.reshape(-1), fmt)
    assert np.array_equal(k.cpu().numpy().reshape(-1), ok.reshape(-1))
    od = oracle.dequantize(oq, ok, fmt, "bf16" if bf16 else "f32").reshape(-1)
    d = fp8.dequantize(q, k, torch.bfloat16 if bf16 else torch.float32)
    assert _vals_equal(bits(d).reshape(-1), od)
    r = fp8.roundtrip(xt, fmt, per_tensor=per_tensor)
    assert _vals_equal(bits(r).reshape(-1), od)
    # recover_exp on the round trip (per row): the oracle's k, or the reference's ValueError
    rk, nbad = oracle.recover_exp(bits(r).reshape(rows, cols), fmt)
    if nbad:
        with pytest.raises(ValueError, match="recipe mismatch"):
            fp8.recover_exp(r, fmt)
    else:
        assert np.array_equal(fp8.recover_exp(r, fmt).cpu().numpy().reshape(-1), rk)


@FUZZ
@given(
    n=st.sampled_from([8, 24, 2048, 2056, 4096 + 8, 3 * 2048 + 16, 65536, 65536 + 24, 200008]),
    bf16=st.booleans(),
    fmt=st.sampled_from(["e4m3", "e5m2"]),
    specials=st.sampled_from([0.0, 0.0, 1e-4, 0.05]),
    offset=st.sampled_from([0, 0, 0, 1, -1, 2, -7, 300]),
    as_tensor=st.booleans(),
    seed=st.integers(0, 2**16),
)
def test_per_tensor_hint_matches_the_oracle(oracle, n, bf16, fmt, specials, offset, as_tensor, seed):
    """fp8.quantize / roundtrip(per_tensor=True, k_hint=...) with the hint
    right, a few off or far out of range, as an int or a device tensor, over
    exponents across the range with NaN, Inf, zeros and subnormals sprinkled
    in: codes, k and the round trip equal the oracle's per-tensor results."""
    from elysium_wan_amd import fp8

    rng = np.random.default_rng(seed)
    e = int(rng.integers(-135, 125))
    x = (rng.standard_normal(n) * np.exp2(float(e))).astype(np.float32)
    if specials:
        pick = rng.random(n) < specials
        pool = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -3e-39, 1e-45], dtype=np.float32)
        x[pick] = pool[rng.integers(0, pool.size, size=int(pick.sum()))]
    if bf16:
        host = oracle.f32_to_bf16_bits(x).reshape(x.shape)
        xt = torch.from_numpy(host.view(np.int16).copy()).view(torch.bfloat16).cuda()
    else:
        host = x
        xt = torch.from_numpy(x.copy()).cuda()
    oq, ok = oracle.quantize(host.reshape(1, -1), fmt)
    hint = int(ok.reshape(-1)[0]) + offset
    h = torch.tensor([hint], dtype=torch.int32, device="cuda") if as_tensor else hint
    say("fp8 hint fuzz", n, "bf16" if bf16 else "f32", fmt, specials, "hint", hint, "k", int(ok.reshape(-1)[0]),
        "tensor" if as_tensor else "int", seed)
    q, k = fp8.quantize(xt, fmt, per_tensor=True, k_hint=h)
    assert _codes_equal(bits(q).reshape(-1), oq.reshape(-1), fmt)
    assert int(k.reshape(-1)[0]) == int(ok.reshape(-1)[0])
    od = oracle.dequantize(oq, ok, fmt, "bf16" if bf16 else "f32").reshape(-1)
    r = fp8.roundtrip(xt, fmt, per_tensor=True, k_hint=h)
    assert _vals_equal(bits(r).reshape(-1), od)
