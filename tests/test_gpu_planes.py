"""The lossless wire codecs on the GPU: the byte-plane wire
(codec/planes.py:141-190) for every wire dtype and the unscaled e4m3
nibble-plane wire (codec/fp8_planes.py:19-52), against the reference's own
payload bytes (tests/golden/planes.npz, zlib-1 containers) and the oracle,
at golden sizes and at C1's boundary size, aligned and not."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden
from gpu_util import activation, bits, say

pytestmark = pytest.mark.gpu

_TORCH = {
    "torch.float32": torch.float32,
    "torch.bfloat16": torch.bfloat16,
    "torch.float16": torch.float16,
    "torch.float8_e4m3fn": torch.float8_e4m3fn,
    "torch.float8_e5m2": torch.float8_e5m2,
    "torch.int64": torch.int64,
}


def _from_bytes(raw: np.ndarray, dtype, shape, device="cuda") -> torch.Tensor:
    return torch.from_numpy(raw.copy()).to(device).view(dtype).reshape(shape)


def _raw(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().reshape(-1).view(torch.uint8).cpu().numpy()


def test_byte_plane_payloads_equal_the_reference_bytes():
    from elysium_wan_amd import planes

    g = golden("planes.npz")
    for name in g["plane_names"]:
        name = str(name)
        dtype = _TORCH[str(g[f"p_{name}_dtype"])]
        shape = tuple(int(s) for s in g[f"p_{name}_shape"])
        t = _from_bytes(g[f"p_{name}_t"], dtype, shape)
        say("byte planes golden", name, shape)
        payload, sh = planes.encode(t)
        assert sh == shape
        assert payload == g[f"p_{name}_payload"].tobytes(), name
        back = planes.decode(payload, shape)
        assert back.dtype == dtype and tuple(back.shape) == shape and back.device.type == "cuda"
        assert np.array_equal(_raw(back), g[f"p_{name}_decoded"]), name


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.int64])
def test_split_and_join_equal_the_oracle_aligned_and_not(oracle, dtype):
    """ely_byteplanes_split through the C ABI against the oracle's byte
    split, on the vector path (aligned, n % 16 == 0) and the element-wise
    path (4 bytes off, odd n); join inverts it."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    gen = torch.Generator().manual_seed(5)
    base = torch.randint(-(1 << 62), 1 << 62, (200_016,), generator=gen, dtype=torch.int64).view(torch.uint8).cuda()
    esz = torch.empty(0, dtype=dtype).element_size()
    for off, n in ((0, 200_000 * 8 // esz), (4, 1001)):
        x = base[off : off + n * esz]
        say("split/join", dtype, "offset", off, "n", n)
        planes = torch.empty(n * esz, dtype=torch.uint8, device="cuda")
        _lib.check(L.ely_byteplanes_split(x.data_ptr(), n, esz, planes.data_ptr(), _lib.stream_ptr(x.device)), "split")
        want = np.concatenate(oracle.byte_planes(x.cpu().numpy(), esz))
        assert np.array_equal(planes.cpu().numpy(), want)
        dst = torch.empty(n * esz + 4, dtype=torch.uint8, device="cuda")[off : off + n * esz]
        _lib.check(L.ely_byteplanes_join(planes.data_ptr(), n, esz, dst.data_ptr(), _lib.stream_ptr(x.device)), "join")
        assert torch.equal(dst, x)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_byte_plane_wire_round_trip_at_c1_size(oracle, dtype):
    """The C1 boundary activation [8, 2048, 2560] crosses the byte-plane wire
    bit for bit; its payload equals the oracle's."""
    from elysium_wan_amd import planes

    x = activation((8, 2048, 2560), seed=51, dtype=dtype)
    say("byte-plane wire C1", dtype)
    payload, shape = planes.encode(x)
    back = planes.decode(payload, shape)
    assert torch.equal(back.view(torch.uint8), x.view(torch.uint8))
    assert payload == oracle.planes_encode(_raw(x), str(dtype).replace("torch.", ""))


def test_nibble_payloads_equal_the_reference_bytes():
    from elysium_wan_amd import fp8_planes

    g = golden("planes.npz")
    for name in g["nibble_names"]:
        name = str(name)
        shape = tuple(int(s) for s in g[f"n_{name}_shape"])
        raw = g[f"n_{name}_t"]
        if "bfloat16" in str(g[f"n_{name}_dtype"]):
            t = torch.from_numpy(raw.view(np.int16).copy()).view(torch.bfloat16).cuda().reshape(shape)
        else:
            t = torch.from_numpy(raw.copy()).cuda().reshape(shape)
        say("nibble planes golden", name, shape)
        payload, sh = fp8_planes.encode(t)
        assert sh == shape
        assert payload == g[f"n_{name}_payload"].tobytes(), name
        back = fp8_planes.decode(payload, shape)
        assert back.dtype == torch.float32
        assert np.array_equal(bits(back).reshape(-1).view(np.uint32), g[f"n_{name}_decoded"].reshape(-1).view(np.uint32))
    for row, refused in zip(g["n_bad_t"], g["n_bad_refused"]):
        if refused:
            with pytest.raises(AssertionError, match="recipe mismatch"):
                fp8_planes.encode(torch.from_numpy(row.copy()).cuda())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_nibble_wire_at_c1_size_and_odd_counts(oracle, dtype):
    """An e4m3-representable C1 boundary tensor: nibble planes equal the
    oracle's, the wire round trip is exact; odd counts and unaligned views
    take the element-wise path; one value off the grid is refused."""
    from elysium_wan_amd import fp8_planes

    gen = torch.Generator().manual_seed(52)
    codes = torch.randint(0, 256, (8, 2048, 2560), generator=gen, dtype=torch.int64)
    codes[(codes & 0x7F) == 0x7F] = 0x3C
    t = codes.to(torch.uint8).view(torch.float8_e4m3fn).to(dtype).cuda()
    for view in (t, t.reshape(-1)[1:100_002]):
        say("nibble wire", dtype, tuple(view.shape))
        payload, shape = fp8_planes.encode(view)
        back = fp8_planes.decode(payload, shape)
        assert torch.equal(back, view.float())
        assert payload == oracle.fp8_planes_encode(bits(view))
    bad = t.reshape(-1)[:4097].clone()
    bad[4096] = 1.0 + 2.0**-5 if dtype == torch.float32 else 1.0 + 2.0**-6
    with pytest.raises(AssertionError):
        fp8_planes.encode(bad)


def test_empty_and_scalar_tensors():
    from elysium_wan_amd import fp8_planes, planes

    for t in (torch.empty(0, device="cuda"), torch.tensor(2.5, device="cuda"), torch.empty(3, 0, dtype=torch.bfloat16, device="cuda")):
        payload, shape = planes.encode(t)
        assert torch.equal(planes.decode(payload, shape), t)
        payload, shape = fp8_planes.encode(t)
        assert torch.equal(fp8_planes.decode(payload, shape), t.float())


def test_f32_planes_wire_at_c1_gradient_size_and_refusals(oracle):
    """codec/f32_planes.py:17-33 at the size of C1's boundary gradient
    ([8, 2048, 2560] fp32, N(0, 1e-4)): payload bytes equal the oracle's,
    decode is bit-exact on the GPU; a non-fp32 tensor is refused with the
    reference's AssertionError and a wrong shape with numpy's ValueError."""
    from elysium_wan_amd import f32_planes

    t = torch.empty(8, 2048, 2560, device="cuda").normal_(0.0, 1e-4, generator=torch.Generator(device="cuda").manual_seed(4))
    say("f32 planes C1 gradient")
    payload, shape = f32_planes.encode(t)
    assert payload == oracle.f32_planes_encode(_raw(t))
    assert len(payload) < t.numel() * 4  # the exponent planes code below raw
    back = f32_planes.decode(payload, shape)
    assert torch.equal(back.view(torch.int32), t.view(torch.int32))
    with pytest.raises(AssertionError):
        f32_planes.encode(t.bfloat16())
    with pytest.raises(ValueError):
        f32_planes.decode(payload, (3, 5))


def test_byte_planes_compress_trained_like_fp32():
    """The reference's test_planes_compresses_trained_like_fp32
    (tests/unit/test_codecs_identity.py:46-49): the exponent planes of
    N(0, 0.02) weights code below the raw bytes."""
    from elysium_wan_amd import planes

    t = torch.empty(4, 64, 256, device="cuda").normal_(0.0, 0.02, generator=torch.Generator(device="cuda").manual_seed(0))
    payload, _ = planes.encode(t)
    assert len(payload) < t.numel() * 4


def test_nibble_encode_counts_every_unrepresentable_element():
    """ely_fp8_nibbles_encode adds one to the bad count per element that is
    not exactly an e4m3 value (ely.h), whichever path takes it: planted
    NaN, Inf, beyond-448 and off-grid elements in the vector path, in the
    element-wise tail and in an unaligned view, against their exact number."""
    from elysium_wan_amd import _lib

    L = _lib.load()
    gen = torch.Generator().manual_seed(21)
    for dtype in (torch.bfloat16, torch.float32):
        for n, off in ((1_000_003, 0), (4_099, 0), (70_001, 1)):
            codes = torch.randint(0, 256, (n,), generator=gen, dtype=torch.int64).to(torch.uint8)
            x = codes.view(torch.float8_e4m3fn).float()
            x = torch.where(torch.isnan(x), torch.zeros_like(x), x)
            idx = torch.randperm(n, generator=gen)[:37]
            planted = torch.tensor([float("nan"), float("inf"), -500.0, 1.0 + 2.0**-6])[torch.arange(37) % 4]
            x[idx] = planted
            buf = torch.zeros(n + off, dtype=dtype, device="cuda")
            t = buf[off:]
            t.copy_(x.to(dtype))
            hi = torch.empty((n + 1) // 2, dtype=torch.uint8, device="cuda")
            lo = torch.empty_like(hi)
            bad = torch.zeros(1, dtype=torch.int64, device="cuda")
            say("nibble bad count", dtype, n, off)
            _lib.check(L.ely_fp8_nibbles_encode(t.data_ptr(), _lib.dtype_code(t), n, hi.data_ptr(), lo.data_ptr(), bad.data_ptr(),
                                                _lib.stream_ptr(t.device)), "nibbles")
            assert int(bad.item()) == 37
