"""recover_exp and the scaled-fp8 wire image on the GPU against the
reference's own outputs (tests/golden: payload bytes made by
codec/planes.py:85-117 with zlib-1, per-row recovered exponents of
model/fp8.py:66-93) and the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden
from gpu_util import activation, bits, f32_equal, from_bits_bf16, say

pytestmark = pytest.mark.gpu


def _tensor(raw, dname_or_dtype):
    if "bf16" in str(dname_or_dtype) or "bfloat16" in str(dname_or_dtype):
        return from_bits_bf16(raw, "cuda")
    return torch.from_numpy(raw.astype(np.float32)).cuda()


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dname", ["f32", "bf16"])
def test_recover_exp_equals_the_reference_golden(fmt, dname):
    from elysium_wan_amd import fp8

    g = golden("fp8_rows.npz")
    pre = f"{fmt}_{dname}"
    for src, kk, ok in (("rt", "rec", "rec_ok"), ("cand", "cand_k", "cand_ok")):
        t = _tensor(g[f"{pre}_{src}"], dname)
        say("recover_exp golden", pre, src, tuple(t.shape))
        want_k, want_ok = g[f"{pre}_{kk}"], g[f"{pre}_{ok}"]
        good = np.nonzero(want_ok)[0]
        k = fp8.recover_exp(t[torch.from_numpy(good).cuda()], fmt)
        assert np.array_equal(bits(k).reshape(-1), want_k[good])
        for r in np.nonzero(want_ok == 0)[0][:8]:
            with pytest.raises(ValueError, match="recipe mismatch"):
                fp8.recover_exp(t[int(r) : int(r) + 1], fmt)


def test_wire_payloads_equal_the_reference_bytes():
    from elysium_wan_amd import planes

    g = golden("wire.npz")
    for name in g["names"]:
        name = str(name)
        fmt = "e5m2" if name.endswith("e5m2") else "e4m3"
        shape = tuple(int(s) for s in g[f"{name}_shape"])
        t = _tensor(g[f"{name}_t"], str(g[f"{name}_dtype"])).reshape(shape)
        say("wire golden", name, shape)
        payload, sh = planes.encode_scaled_fp8(t, fmt)
        assert sh == shape
        assert payload == g[f"{name}_payload"].tobytes(), name
        out = planes.decode(payload, shape)
        assert f32_equal(bits(out).reshape(-1), g[f"{name}_decoded"].reshape(-1))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_wire_round_trip_of_a_c1_activation_and_its_refusal(oracle, fmt):
    """tests/unit/test_codecs_identity.py:59-68 at C1's boundary shape: the
    recipe's round trip crosses the wire exactly; an un-narrowed tensor is
    refused."""
    from elysium_wan_amd import fp8, planes

    x = activation((8, 2048, 2560), seed=21 if fmt == "e4m3" else 22)
    rt = fp8.roundtrip(x, fmt)
    say("wire C1", fmt)
    payload, shape = planes.encode_scaled_fp8(rt, fmt)
    back = planes.decode(payload, shape)
    assert torch.equal(back, rt.float())
    k = fp8.recover_exp(rt, fmt)
    ok, bad = oracle.recover_exp(bits(rt[0, :64]), fmt)
    assert bad == 0 and np.array_equal(bits(k[0, :64]).reshape(-1), ok)
    with pytest.raises(ValueError, match="recipe mismatch"):
        planes.encode_scaled_fp8(x, fmt)


def test_gradient_scale_values_survive_the_wire():
    """test_codecs_identity.py:62: randn * 1e-4, values an unscaled cast zeroes."""
    from elysium_wan_amd import fp8, planes

    x = torch.randn(3, 8, 32, device="cuda") * 1e-4
    for fmt in ("e4m3", "e5m2"):
        q = fp8.roundtrip(x, fmt)
        assert float(q.abs().sum()) > 0
        payload, shape = planes.encode_scaled_fp8(q, fmt)
        assert torch.equal(planes.decode(payload, shape), q)
        with pytest.raises(ValueError):
            planes.encode_scaled_fp8(x, fmt)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [(5, 1001), (1, 100_000), (64, 8200)])
def test_recover_exp_on_odd_and_long_rows_equals_the_oracle(oracle, fmt, shape):
    """Element-wise rows (1001 is no multiple of the vector), one long row
    over many segments, and rows past the register path: the exponents and
    the byte image equal the oracle's, and rows off the fp8 grid are
    refused."""
    from elysium_wan_amd import _lib, fp8

    x = activation(shape, seed=shape[1] % 97)
    rt = fp8.roundtrip(x, fmt)
    say("recover odd/long", fmt, shape)
    k = fp8.recover_exp(rt, fmt)
    ok, bad = oracle.recover_exp(bits(rt), fmt)
    assert bad == 0 and np.array_equal(bits(k).reshape(-1), ok)
    q = torch.empty(shape, dtype=torch.uint8, device="cuda")
    L = _lib.load()
    _lib.check(L.ely_fp8_quantize_k(rt.data_ptr(), _lib.BF16, shape[0], shape[1], _lib.FMT[fmt], k.data_ptr(), q.data_ptr(), _lib.stream_ptr(rt.device)), "quantize_k")
    # the byte image with the recovered exponents: each product is exact
    xf = oracle.bf16_bits_to_f32(bits(rt)).reshape(shape).astype(np.float64)
    kk = bits(k).reshape(-1).astype(np.float64)
    oq = oracle.fp8_encode((xf * np.exp2(-kk)[:, None]).astype(np.float32), fmt)
    assert np.array_equal(q.cpu().numpy(), oq)
    # one value with a 6-bit mantissa in row 0: no candidate exponent makes it fp8
    off = rt.clone()
    off[0, shape[1] // 2] = (1 + 2.0**-6) * 2.0 ** int(bits(k).reshape(-1)[0])
    with pytest.raises(ValueError, match="recipe mismatch"):
        fp8.recover_exp(off, fmt)


def _oracle_image(oracle, t_bits, fmt):
    """The reference's byte image and int8 exponents (codec/planes.py:85-117),
    unpacked from the oracle's payload."""
    import struct
    import zlib

    payload = oracle.wire_encode(t_bits, fmt)
    off = struct.calcsize("<BBQ")
    lv, lk = struct.unpack_from("<II", payload, off)
    off += 8
    q = np.frombuffer(zlib.decompress(payload[off : off + lv]), dtype=np.uint8)
    k = np.frombuffer(zlib.decompress(payload[off + lv : off + lv + lk]), dtype=np.int8)
    return q, k


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dname", ["bf16", "f32"])
@pytest.mark.parametrize("cols", [32, 768, 2560, 8192, 1000])
def test_recover_image_equals_the_oracle(oracle, fmt, dname, cols):
    """ely_fp8_recover_image (k and the byte image in one call; one pass over
    rows that fit registers, the multi-launch path otherwise) on rows taking
    each branch: an ordinary round trip, a zero row, a tiny and a huge row
    (base exponent off the instruction path), a row whose base exponent is
    one too high (offset -1 wins), and for e5m2 a row holding +-Inf and an
    all-Inf row (|x|max not finite).  k,
    the bytes and the int8 exponents equal the oracle's wire_encode; a value
    off the grid is refused with the reference's message."""
    from elysium_wan_amd import _lib, fp8, planes

    dt = {"bf16": torch.bfloat16, "f32": torch.float32}[dname]
    g = torch.Generator().manual_seed(cols)
    x = torch.randn(7, cols, generator=g)
    x[1] = 0.0
    # |base| > 108: the candidates leave the instruction path (restatement rows)
    x[2] *= 2.0 ** (-118 if fmt == "e4m3" else -100)
    x[3] *= 2.0 ** (115 if fmt == "e4m3" else 121)
    x[4, 0] = 255.9  # rounds to 256 in fp8: the base exponent is one octave high
    if fmt == "e5m2":
        x[5, cols // 2] = float("inf")
        x[5, cols - 1] = float("-inf")
        x[6] *= 2.0**-118  # 2^-k overflows in the quantize: the round trip is all +-Inf
    rt = fp8.roundtrip(x.to(dt).cuda(), fmt)
    rows = rt.shape[0]
    say("recover_image", fmt, dname, cols)
    k = torch.empty(rows, dtype=torch.int32, device="cuda")
    q = torch.empty(rt.shape, dtype=torch.uint8, device="cuda")
    bad = torch.zeros(1, dtype=torch.int64, device="cuda")
    L = _lib.load()
    ws = _lib.workspace(rt.device, L.ely_fp8_recover_workspace_bytes(rows))
    _lib.check(L.ely_fp8_recover_image(rt.data_ptr(), _lib.dtype_code(rt), rows, cols, _lib.FMT[fmt], k.data_ptr(), q.data_ptr(),
                                       bad.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(rt.device)), "recover_image")
    assert int(bad.item()) == 0
    ok, obad = oracle.recover_exp(bits(rt), fmt)
    assert obad == 0 and np.array_equal(bits(k), ok)
    oq, ok8 = _oracle_image(oracle, bits(rt), fmt)
    assert np.array_equal(q.cpu().numpy().reshape(-1), oq)
    assert np.array_equal(bits(k).astype(np.int8), ok8)
    # recover_exp (register path without the image) agrees
    assert torch.equal(fp8.recover_exp(rt, fmt).reshape(-1), k)
    off = rt.clone()
    off[0, cols // 3] = (1 + 2.0**-6) * 2.0 ** int(bits(k)[0])
    with pytest.raises(ValueError, match="^boundary tensor is not scaled-FP8 representable: recipe mismatch$"):
        planes.encode_scaled_fp8(off, fmt)


def test_encoders_take_host_tensors_as_the_reference_does():
    """The reference's encoders copy their input to the host first, so any
    device's tensor goes in (codec/planes.py:87, 143; fp8_planes.py:21;
    f32_planes.py:19): a host tensor here is copied to the GPU and gives
    the same payload as the same tensor on the GPU."""
    from elysium_wan_amd import f32_planes, fp8, fp8_planes, planes

    gen = torch.Generator().manual_seed(12)
    x = torch.randn(6, 40, generator=gen)
    scaled = fp8.roundtrip(x.cuda().bfloat16()).cpu()  # a tensor that is its own scaled-fp8 round trip
    e4m3 = x.to(torch.float8_e4m3fn).float()  # every element an e4m3 value
    say("wire encoders on host tensors")
    for enc, t in ((planes.encode, x.bfloat16()), (planes.encode, x), (planes.encode_scaled_fp8, scaled),
                   (fp8_planes.encode, e4m3), (f32_planes.encode, x)):
        assert t.device.type == "cpu"
        assert enc(t) == enc(t.cuda())
