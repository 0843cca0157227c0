"""Per-tensor fp8 quantize with an exponent hint (fp8.quantize(...,
per_tensor=True, k_hint=...), ely_fp8_quantize_hint): whatever the hint, the
bytes and the exponent are model/fp8.py:28-49's for one row of every
element, checked against the oracle, against the split path and against
torch's own ops on the GPU at config C4's full size; the device flag says
whether the one pass stood (hint right) or the fixup pass ran (hint wrong,
out of range, or a tensor with no one-pass form)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import activation, bits, f32_equal, say

pytestmark = pytest.mark.gpu


def _oracle_in(x: torch.Tensor) -> np.ndarray:
    return bits(x) if x.dtype == torch.bfloat16 else bits(x).astype(np.float32)


def _hint_call(x: torch.Tensor, fmt: str, k_hint: int, want_q=True, want_out=False, device_hint=False, alias=False):
    """ely_fp8_quantize_hint through the C ABI: (q, k, out, hit).  device_hint:
    the hint from device memory; alias: that word is also the k output."""
    from elysium_wan_amd import _lib, fp8

    L = _lib.load()
    x = x.contiguous()
    n = x.numel()
    q = torch.full((n,), 0xA5, dtype=torch.uint8, device=x.device) if want_q else None
    out = torch.full((n,), float("nan"), dtype=x.dtype, device=x.device) if want_out else None
    k = torch.full((1,), -777, dtype=torch.int32, device=x.device)
    hdev = None
    if device_hint:
        hdev = k if alias else torch.empty(1, dtype=torch.int32, device=x.device)
        hdev.fill_(k_hint)
    hit = torch.full((1,), -1, dtype=torch.int32, device=x.device)
    ws = torch.empty(L.ely_fp8_hint_workspace_bytes(n), dtype=torch.uint8, device=x.device)
    _lib.check(L.ely_fp8_quantize_hint(x.data_ptr(), _lib.dtype_code(x), n, _lib.FMT[fmt], 12345 if device_hint else k_hint,
                                       None if hdev is None else hdev.data_ptr(), None if q is None else q.data_ptr(), k.data_ptr(),
                                       None if out is None else out.data_ptr(), hit.data_ptr(), ws.data_ptr(), ws.numel(),
                                       _lib.stream_ptr(x.device)), "quantize_hint")
    torch.cuda.synchronize()
    assert fp8.FORMATS[fmt]
    return q, int(k.item()), out, int(hit.item())


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [8, 2048, 2056, 65536 + 8, 3 * 2048 * 257])
def test_hit_and_miss_equal_the_oracle(oracle, fmt, dtype, n):
    """Hints equal to the exponent (one pass), one and five off (fixup), and
    out of the one-pass range: the same bytes and exponent as the oracle's
    per-tensor quantize, and the flag telling which pass stood."""
    x = activation((n,), seed=300 + n % 97, dtype=dtype)
    oq, ok = oracle.quantize(_oracle_in(x.reshape(1, -1)), fmt)
    k_true = int(ok.reshape(-1)[0])
    for hint in (k_true, k_true + 1, k_true - 1, k_true + 5, 200, -200):
        say("fp8 hint", fmt, dtype, n, "hint", hint, "k", k_true)
        q, k, _, hit = _hint_call(x, fmt, hint)
        assert k == k_true
        assert np.array_equal(bits(q), oq.reshape(-1)), f"fp8 bytes, hint {hint}"
        assert hit == (1 if hint == k_true else 0)


@pytest.mark.parametrize("alias", [False, True])
def test_device_hint_read_on_the_gpu(oracle, alias):
    """The hint from device memory (the int argument is then ignored: a wrong
    one is passed), also when that word is the k output itself (the last
    step's exponent updated in place): right, off and out-of-range hints
    give the oracle's bytes and k, and the flag says which pass stood."""
    x = activation((3 * 2048 * 33,), seed=331)
    for fmt in ("e4m3", "e5m2"):
        oq, ok = oracle.quantize(_oracle_in(x.reshape(1, -1)), fmt)
        k_true = int(ok.reshape(-1)[0])
        for hint in (k_true, k_true + 1, k_true - 3, 150):
            say("fp8 device hint", fmt, "alias" if alias else "separate", hint, "k", k_true)
            q, k, _, hit = _hint_call(x, fmt, hint, device_hint=True, alias=alias)
            assert k == k_true
            assert np.array_equal(bits(q), oq.reshape(-1))
            assert hit == (1 if hint == k_true else 0)


def test_steps_with_the_last_exponent_as_the_hint():
    """A boundary quantized every step with the previous step's k tensor as
    the hint (fp8.quantize(..., k_hint=k_prev)): every step equals the
    hint-free per-tensor quantize, whether the scale held or moved."""
    from elysium_wan_amd import fp8

    k_prev = None
    for step, scale in enumerate((1.0, 1.3, 1.3, 5.0, 0.2, 0.2)):
        x = (activation((8, 4096), seed=500 + step) * scale).to(torch.bfloat16)
        say("fp8 hint steps", step, scale)
        q, k = fp8.quantize(x, "e4m3", per_tensor=True, k_hint=k_prev)
        qw, kw = fp8.quantize(x, "e4m3", per_tensor=True)
        assert torch.equal(q.view(torch.uint8), qw.view(torch.uint8)) and torch.equal(k, kw)
        k_prev = k.reshape(1) if k_prev is None or step % 2 else k.reshape(1).clone()


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_round_trip_with_a_hint_equals_the_round_trip(fmt):
    from elysium_wan_amd import fp8

    x = activation((16, 4096), seed=41)
    want = fp8.roundtrip(x, fmt, per_tensor=True)
    k = int(fp8.scale_exp(x, fmt, per_tensor=True).reshape(-1)[0])
    for hint in (k, k - 2):
        say("fp8 hint round trip", fmt, hint)
        got = fp8.roundtrip(x, fmt, per_tensor=True, k_hint=hint)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        q, kk, out, hit = _hint_call(x, fmt, hint, want_q=False, want_out=True)
        assert kk == k and hit == (1 if hint == k else 0)
        assert torch.equal(out.view(torch.int16), want.reshape(-1).view(torch.int16))


def test_no_one_pass_form_falls_back_exactly(oracle):
    """n not a whole number of 16-byte vectors, an unaligned view, Inf and NaN
    (|x|max not finite: the exact-arithmetic path), an all-zero tensor and an
    empty one: the split path's results, and the flag 0."""
    from elysium_wan_amd import fp8

    base = activation((4096 + 24,), seed=43)
    cases = {
        "ragged": activation((4099,), seed=44),
        "unaligned": base[3:3 + 4096],
        "inf": torch.cat([activation((4095,), seed=45), torch.tensor([float("inf")], dtype=torch.bfloat16, device="cuda")]),
        "nan": torch.cat([torch.tensor([float("nan")], dtype=torch.bfloat16, device="cuda"), activation((4095,), seed=46)]),
        "zeros": torch.zeros(4096, dtype=torch.bfloat16, device="cuda"),
    }
    for name, x in cases.items():
        for fmt in ("e4m3", "e5m2"):
            say("fp8 hint fallback", name, fmt)
            oq, ok = oracle.quantize(_oracle_in(x.reshape(1, -1)), fmt)
            k_true = int(ok.reshape(-1)[0])
            for hint in (k_true, 0, 3):
                q, k = fp8.quantize(x, fmt, per_tensor=True, k_hint=hint)
                assert int(k.reshape(-1)[0]) == k_true
                assert np.array_equal(bits(q).reshape(-1), oq.reshape(-1)), (name, fmt, hint)
    for name in ("ragged", "unaligned"):
        _, _, _, hit = _hint_call(cases[name], "e4m3", 0)
        assert hit == 0
    q, k = fp8.quantize(torch.empty(0, dtype=torch.bfloat16, device="cuda"), "e4m3", per_tensor=True, k_hint=4)
    assert q.numel() == 0 and int(k.reshape(-1)[0]) == 0


def test_hint_argument_checks():
    from elysium_wan_amd import fp8

    x = activation((64,), seed=47)
    with pytest.raises(ValueError, match="per-tensor"):
        fp8.quantize(x, "e4m3", k_hint=0)
    with pytest.raises(ValueError, match="int32"):
        fp8.quantize(x, "e4m3", per_tensor=True, k_hint=2**40)
    with pytest.raises(ValueError, match="one int32"):
        fp8.quantize(x, "e4m3", per_tensor=True, k_hint=torch.zeros(2, dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError, match="one int32"):
        fp8.quantize(x, "e4m3", per_tensor=True, k_hint=torch.zeros(1, dtype=torch.int64, device="cuda"))


GUESS_STRIDE, SEG_ELEMS = 61, 2048  # the sampled guess reads segments 0, 61, 122, ... of 2,048 elements


def _guess_call(x: torch.Tensor, fmt: str, ws_bytes=None, roundtrip=False):
    """ely_fp8_quantize (or ely_fp8_roundtrip with no q and no k) of x as one
    row, with a workspace of ws_bytes (default: what ely_fp8_workspace_bytes
    asks): (q, k, out, workspace)."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    n = x.numel()
    dt = _lib.dtype_code(x)
    need = L.ely_fp8_workspace_bytes(1, n, dt)
    ws = torch.zeros(need if ws_bytes is None else ws_bytes, dtype=torch.uint8, device=x.device)
    sp = _lib.stream_ptr(x.device)
    if roundtrip:
        out = torch.full_like(x, float("nan"))
        _lib.check(L.ely_fp8_roundtrip(x.data_ptr(), dt, 1, n, _lib.FMT[fmt], out.data_ptr(), None, None, ws.data_ptr(), ws.numel(), sp), "roundtrip")
        torch.cuda.synchronize()
        return None, None, out, ws
    q = torch.full((n,), 0xA5, dtype=torch.uint8, device=x.device)
    k = torch.full((1,), -777, dtype=torch.int32, device=x.device)
    _lib.check(L.ely_fp8_quantize(x.data_ptr(), dt, 1, n, _lib.FMT[fmt], q.data_ptr(), k.data_ptr(), ws.data_ptr(), ws.numel(), sp), "quantize")
    torch.cuda.synchronize()
    return q, int(k.item()), None, ws


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("where", ["sampled", "unsampled", "nan sampled", "inf unsampled"])
def test_sampled_guess_equals_the_oracle_and_the_split_path(oracle, fmt, dtype, where):
    """A per-tensor row of 64 MiB takes the sampled guess: the exponent of
    the |x|max of every 61st 2,048-element segment, then the hint path.  A
    -8192 outlier in a sampled segment makes the guess right (one pass); in an
    unsampled one, wrong (the fixup pass); a NaN in the sample, or an Inf
    outside it, leaves the row off the instruction path, so the fixup
    converts it element by element.  Either way the bytes and k are
    the oracle's and the split path's (the same call given too small a
    workspace for the guess), and the word the guess left in the workspace
    is the sample's |x|max, so the sampling itself is checked."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    n = (64 << 20) // (2 if dtype == torch.bfloat16 else 4)
    x = activation((n,), seed=700 + n % 89, dtype=dtype)
    seg = GUESS_STRIDE * 7 if where in ("sampled", "nan sampled") else GUESS_STRIDE * 7 + 3
    x[seg * SEG_ELEMS + 5] = {"sampled": -8192.0, "unsampled": -8192.0, "nan sampled": float("nan"), "inf unsampled": float("inf")}[where]
    say("fp8 sampled guess", fmt, dtype, where)
    oq, ok = oracle.quantize(_oracle_in(x.reshape(1, -1)), fmt)
    q, k, _, ws = _guess_call(x, fmt)
    assert k == int(ok.reshape(-1)[0])
    assert np.array_equal(bits(q), oq.reshape(-1))
    off = L.ely_fp8_hint_workspace_bytes(n)
    if where in ("sampled", "unsampled"):
        sample = x.float().reshape(-1, SEG_ELEMS)[::GUESS_STRIDE].abs().max()
        assert int(ws[off:off + 4].view(torch.int32).item()) == int(sample.reshape(1).view(torch.int32).item())
        assert (float(sample) == 8192.0) == (where == "sampled")
    elif where == "nan sampled":
        assert torch.isnan(ws[off:off + 4].view(torch.float32)).item()
    # the split path: a workspace too small for the guess
    q2, k2, _, _ = _guess_call(x, fmt, ws_bytes=L.ely_fp8_workspace_bytes(2, n, _lib.dtype_code(x)))
    assert k2 == k and torch.equal(q2, q)
    # the round trip, with neither q nor k asked for
    _, _, out, _ = _guess_call(x, fmt, roundtrip=True)
    ort = oracle.roundtrip(_oracle_in(x.reshape(1, -1)), fmt).reshape(-1)
    if dtype == torch.bfloat16:
        assert np.array_equal(bits(out), ort)
    else:
        assert f32_equal(bits(out), ort)


def _c4_activation(seed: int) -> torch.Tensor:
    """Config C4's activation [16, 4096, 8192] bf16: Student-t (df = 3) with
    0.01% of the elements set to +-1e4."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    shape = (16, 4096, 8192)
    z = torch.empty(shape, device="cuda").normal_(generator=g)
    c = torch.zeros(shape, device="cuda")
    for _ in range(3):
        c.add_(torch.empty(shape, device="cuda").normal_(generator=g).square_())
    z.div_(c.div_(3.0).sqrt_())
    del c
    n = z.numel()
    idx = torch.randint(0, n, (n // 10000,), generator=g, device="cuda")
    sign = torch.randint(0, 2, idx.shape, generator=g, device="cuda").float() * 2 - 1
    z.view(-1)[idx] = 1e4 * sign
    return z.to(torch.bfloat16)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_c4_per_tensor_with_a_hint_equals_torch_on_the_gpu(fmt):
    """Config C4's activation at full size, per-tensor, hint right and hint
    wrong: bytes and exponent equal torch's own ops on the GPU running
    model/fp8.py:28-49's arithmetic."""
    from elysium_wan_amd import fp8

    x = _c4_activation(63 if fmt == "e4m3" else 64)
    dt, ebias = fp8.FORMATS[fmt]
    amax = x.abs().amax()
    kt = int(torch.frexp(amax).exponent) - ebias
    qt = (x * torch.exp2(torch.tensor(-kt, dtype=torch.bfloat16, device="cuda"))).to(dt).view(torch.uint8)
    for hint in (kt, kt + 1):
        say("fp8 C4 per-tensor hint", fmt, hint, "k", kt)
        q, k = fp8.quantize(x, fmt, per_tensor=True, k_hint=hint)
        assert int(k.reshape(-1)[0]) == kt
        assert torch.equal(q.view(torch.uint8), qt)
        del q
