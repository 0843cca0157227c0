"""fp8 boundary codec on the GPU (elysium_wan_amd.fp8 -> libelyhip.so) against
the oracle, the reference's golden vectors and torch-on-GPU: fp8 bytes,
exponents and dequantized values bit for bit (model/fp8.py:28-63)."""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from conftest import golden
from gpu_util import activation, bits, f32_equal, from_bits_bf16, say

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _oracle_in(x: torch.Tensor) -> np.ndarray:
    return bits(x) if x.dtype == torch.bfloat16 else bits(x).astype(np.float32)


def _check_against_oracle(oracle, x: torch.Tensor, fmt: str, per_tensor=False):
    from elysium_wan_amd import fp8

    xs = x.reshape(1, -1) if per_tensor else x
    q, k = fp8.quantize(x, fmt, per_tensor=per_tensor)
    oq, ok = oracle.quantize(_oracle_in(xs), fmt)
    assert np.array_equal(bits(q).reshape(-1), oq.reshape(-1)), "fp8 bytes"
    assert np.array_equal(bits(k).reshape(-1), ok.reshape(-1)), "exponents"
    for out_dt, name in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        d = fp8.dequantize(q, k, out_dt)
        od = oracle.dequantize(oq, ok, fmt, name)
        if name == "f32":
            assert f32_equal(bits(d).reshape(-1), od.reshape(-1)), "dequantize f32"
        else:
            assert np.array_equal(bits(d).reshape(-1), od.reshape(-1)), "dequantize bf16"
    rt = fp8.roundtrip(x, fmt, per_tensor=per_tensor)
    ort = oracle.roundtrip(_oracle_in(xs), fmt)
    if x.dtype == torch.bfloat16:
        assert np.array_equal(bits(rt).reshape(-1), ort.reshape(-1)), "roundtrip bf16"
    else:
        assert f32_equal(bits(rt).reshape(-1), ort.reshape(-1)), "roundtrip f32"
    assert torch.equal(bits_t(rt), bits_t(fp8.dequantize(q, k, x.dtype))), "fused roundtrip == quantize+dequantize"


def bits_t(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dname", ["bf16", "f32"])
@pytest.mark.parametrize(
    "shape",
    [(4, 1024, 768), (16, 2560), (7, 8192), (3, 4096 + 8), (6, 4096), (5, 3200), (5, 1000), (3, 7), (2, 1), (9, 16384 + 24),
     (1, 3 * 65536 + 5)],
)
def test_quantize_dequantize_roundtrip_equal_the_oracle(oracle, fmt, dname, shape):
    say("fp8 vs oracle", fmt, dname, shape)
    x = activation(shape, seed=zlib.crc32(repr((fmt, dname, shape)).encode()) % 1000, dtype=DT[dname])
    _check_against_oracle(oracle, x, fmt)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_per_tensor_scaling_equals_the_oracle(oracle, fmt):
    say("fp8 per-tensor", fmt)
    x = activation((4, 1024, 768), seed=3)  # config C0's activation, one exponent
    _check_against_oracle(oracle, x, fmt, per_tensor=True)


def test_unaligned_and_strided_inputs(oracle):
    """A row view that starts off a 16-byte boundary takes the element path."""
    base = activation((4 * 777 + 3,), seed=5)
    x = base[3:].reshape(4, 777)
    say("fp8 unaligned", x.data_ptr() % 16)
    _check_against_oracle(oracle, x, "e4m3")
    t = activation((64, 96), seed=6).t()  # non-contiguous: made contiguous first
    _check_against_oracle(oracle, t, "e5m2")


def test_extreme_rows_equal_torch_on_the_gpu(oracle):
    """Rows whose scale 2^-k or 2^k leaves the dtype's range (subnormal rows,
    huge rows), NaN and Inf rows: the kernels' exact-arithmetic path against
    the reference's own torch expressions evaluated on this GPU, NaN signs
    included (model/fp8.py:28-53)."""
    from elysium_wan_amd import fp8

    g = golden("fp8_rows.npz")
    for fmt, tdt in (("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)):
        for dname in ("bf16", "f32"):
            pre = f"{fmt}_{dname}"
            for key in ("x", "sx"):
                raw = g[f"{pre}_{key}"]
                x = from_bits_bf16(raw, "cuda") if dname == "bf16" else torch.from_numpy(raw.astype(np.float32)).cuda()
                say("fp8 extreme rows", pre, key)
                _, eb = fp8.FORMATS[fmt]
                amax = x.abs().amax(dim=-1, keepdim=True)
                _, e = torch.frexp(amax)
                kref = torch.where(amax > 0, (e - eb).to(torch.int32), torch.zeros_like(e, dtype=torch.int32))
                qref = (x * torch.exp2((-kref).to(x.dtype))).to(tdt)
                dref = qref.to(x.dtype) * torch.exp2(kref.to(x.dtype))
                q, k = fp8.quantize(x, fmt)
                assert torch.equal(k, kref)
                assert np.array_equal(bits(q), bits(qref))
                d = fp8.dequantize(q, k, x.dtype)
                if dname == "bf16":
                    assert np.array_equal(bits(d), bits(dref))
                else:
                    assert f32_equal(bits(d), bits(dref))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dname", ["bf16", "f32"])
@pytest.mark.parametrize("cols", [3200, 4104, 8192])
def test_extreme_rows_on_the_block_row_path(fmt, dname, cols):
    """Rows long enough to be shared by a block's waves (more than 6 vectors
    per lane), each taking another branch: an ordinary row, a NaN, an Inf,
    a row whose 2^-k leaves the instruction path (|x|max ~ 1e38), a tiny
    row (|x|max ~ 1e-38), an all-zero row, and a row whose maximum sits in
    the last wave's part.  k, bytes and the decode equal the reference's
    torch expressions (model/fp8.py:28-53) on this GPU."""
    from elysium_wan_amd import fp8

    tdt = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}[fmt]
    x = activation((7, cols), seed=cols % 97, dtype=torch.float32).float()
    x[1, cols // 3] = float("nan")
    x[2, cols - 5] = float("-inf")
    x[3] *= 5e35
    x[4] *= 1e-39
    x[5] = 0.0
    x[6, cols - 1] = 3000.0
    x = x.to(DT[dname])
    say("fp8 block-row extremes", fmt, dname, cols)
    _, eb = fp8.FORMATS[fmt]
    amax = x.abs().amax(dim=-1, keepdim=True)
    _, e = torch.frexp(amax)
    kref = torch.where(amax > 0, (e - eb).to(torch.int32), torch.zeros_like(e, dtype=torch.int32))
    qref = (x * torch.exp2((-kref).to(x.dtype))).to(tdt)
    dref = qref.to(x.dtype) * torch.exp2(kref.to(x.dtype))
    q, k = fp8.quantize(x, fmt)
    assert torch.equal(k, kref)
    assert np.array_equal(bits(q), bits(qref))
    d = fp8.dequantize(q, k, x.dtype)
    if dname == "bf16":
        assert np.array_equal(bits(d), bits(dref))
    else:
        assert f32_equal(bits(d), bits(dref))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("dname", ["f32", "bf16"])
def test_reference_golden_rows_on_the_gpu(fmt, dname):
    """The reference's own outputs (made on x86) through the GPU path; a NaN
    made inside the arithmetic is compared as NaN (its sign is the device's)."""
    from elysium_wan_amd import fp8

    g = golden("fp8_rows.npz")
    pre = f"{fmt}_{dname}"
    raw = g[f"{pre}_x"]
    x = from_bits_bf16(raw, "cuda") if dname == "bf16" else torch.from_numpy(raw.astype(np.float32)).cuda()
    say("fp8 golden rows", pre)
    q, k = fp8.quantize(x, fmt)
    assert np.array_equal(bits(k).reshape(-1), g[f"{pre}_qk"])
    qb, want = bits(q), g[f"{pre}_q"]
    nan = ((qb & 0x7F) == 0x7F) if fmt == "e4m3" else ((qb & 0x7F) > 0x7C)
    nanw = ((want & 0x7F) == 0x7F) if fmt == "e4m3" else ((want & 0x7F) > 0x7C)
    assert np.array_equal(nan, nanw) and np.array_equal(qb[~nan], want[~nanw])
    d = fp8.dequantize(q, k)
    assert f32_equal(bits(d), g[f"{pre}_deq_f32"])


def test_full_size_activation_c1_properties(oracle):
    """Config C1's activation [8, 2048, 2560] (e4m3) and gradient (e5m2):
    fused == unfused, every fp8-normal element within half an fp8 ulp of x,
    and 512 seeded rows bit-identical to the oracle."""
    from elysium_wan_amd import fp8

    for fmt, seed, mant in (("e4m3", 11, 3), ("e5m2", 12, 2)):
        say("fp8 C1 full size", fmt)
        x = activation((8, 2048, 2560), seed=seed)
        q, k = fp8.quantize(x, fmt)
        rt = fp8.roundtrip(x, fmt)
        assert torch.equal(bits_t(rt), bits_t(fp8.dequantize(q, k, torch.bfloat16)))
        xf, rf = x.float(), rt.float()
        scale = torch.exp2(k.float())
        normal = xf.abs() >= scale * (2.0 ** (-6 if fmt == "e4m3" else -14))
        err = ((rf - xf).abs() / xf.abs().clamp_min(1e-30))[normal]
        assert float(err.max()) <= 2.0 ** -(mant + 1) * (1 + 1e-6)
        rows = torch.randperm(16384, generator=torch.Generator().manual_seed(seed))[:512]
        xr = x.reshape(16384, 2560)[rows.cuda()]
        oq, ok = oracle.quantize(bits(xr), fmt)
        assert np.array_equal(bits(q.reshape(16384, 2560)[rows.cuda()]), oq)
        assert np.array_equal(bits(k.reshape(-1)[rows.cuda()]), ok)


def test_scale_exp_is_the_quantize_exponent():
    from elysium_wan_amd import fp8

    x = activation((33, 2560), seed=13)
    _, k = fp8.quantize(x, "e4m3")
    assert torch.equal(fp8.scale_exp(x, "e4m3"), k)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("cols", [16, 1008, 1024, 1040, 2560, 3072, 8192 + 16])
def test_dequantize_every_code_with_a_distinct_exponent_per_row(oracle, fmt, cols):
    """Codes cycling through all 256 bytes (NaN and Inf codes included) and an
    exponent per row drawn from [-140, 140] (both of the kernel's paths, and
    results that overflow or go subnormal), neighbours always different: a
    value taken with its neighbour row's exponent, where a wave's 1,024 codes
    cross a row boundary, changes the bytes.  bf16 and fp32 out, vs the oracle."""
    from elysium_wan_amd import fp8

    rows = max(3, (3 * 4096 + cols - 1) // cols)
    rng = np.random.default_rng(cols)
    codes = ((np.arange(rows * cols, dtype=np.int64) * 37 + rng.integers(0, 256)) % 256).astype(np.uint8)
    kk = rng.integers(-140, 141, rows).astype(np.int32)
    for r in range(1, rows):
        if kk[r] == kk[r - 1]:
            kk[r] += 1
    q = torch.from_numpy(codes.reshape(rows, cols)).cuda().view(fp8.FORMATS[fmt][0])
    k = torch.from_numpy(kk.reshape(rows, 1)).cuda()
    for out_dt, name in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        say("fp8 dequantize distinct exponents", fmt, cols, name)
        d = bits(fp8.dequantize(q, k, out_dt)).reshape(-1)
        od = oracle.dequantize(codes.reshape(rows, cols), kk, fmt, name).reshape(-1)
        assert f32_equal(d, od) if name == "f32" else np.array_equal(d, od)


def test_empty_inputs():
    from elysium_wan_amd import fp8

    x = torch.empty(0, 64, dtype=torch.bfloat16, device="cuda")
    q, k = fp8.quantize(x)
    assert q.shape == (0, 64) and k.shape == (0, 1)
    assert fp8.dequantize(q, k).shape == (0, 64)
    z = torch.empty(3, 0, dtype=torch.bfloat16, device="cuda")
    q, k = fp8.quantize(z)
    assert k.shape == (3, 1) and int(k.abs().sum()) == 0


def test_long_rows_beyond_the_partial_budget(oracle):
    """More long rows (cols > 8192) than the partial-max launch has waves:
    one wave per row strides over its segments."""
    x = activation((9000, 8200), seed=12)
    say("fp8 9000 long rows")
    _check_against_oracle(oracle, x, "e4m3")


def _c4_activation(seed: int) -> torch.Tensor:
    """Config C4's activation [16, 4096, 8192] bf16: Student-t (df = 3) with
    0.01% of the elements set to +-1e4, generated on the GPU."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    shape = (16, 4096, 8192)
    z = torch.randn(shape, generator=g, device="cuda")
    c = torch.zeros(shape, device="cuda")
    for _ in range(3):
        c.add_(torch.randn(shape, generator=g, device="cuda").square_())
    z.div_(c.div_(3.0).sqrt_())
    del c
    n = z.numel()
    idx = torch.randint(0, n, (n // 10000,), generator=g, device="cuda")
    sign = torch.randint(0, 2, idx.shape, generator=g, device="cuda").float() * 2 - 1
    z.view(-1)[idx] = 1e4 * sign
    return z.to(torch.bfloat16)


def _c4_gradient(seed: int) -> torch.Tensor:
    """Config C4's gradient [16, 4096, 8192] bf16 drawn N(0, 1e-5)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.empty((16, 4096, 8192), device="cuda").normal_(0.0, 1e-5, generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("which", ["activation", "gradient"])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_c4_per_row_and_per_tensor_equal_torch_on_the_gpu(fmt, which):
    """Config C4 at full size, the Student-t activation and the N(0, 1e-5)
    gradient: bytes and exponents of per-row and per-tensor scaling equal
    torch's own ops on the GPU running model/fp8.py:28-49's arithmetic
    (frexp of |x|max, the pow2 product in bf16, torch's fp8 conversion);
    decode is exact."""
    from elysium_wan_amd import fp8

    seed = (61 if fmt == "e4m3" else 62) + (0 if which == "activation" else 10)
    x = _c4_activation(seed) if which == "activation" else _c4_gradient(seed)
    dt, ebias = fp8.FORMATS[fmt]
    for per_tensor in (False, True):
        say("fp8 C4", which, fmt, "per-tensor" if per_tensor else "per-row")
        q, k = fp8.quantize(x, fmt, per_tensor=per_tensor)
        xs = x.reshape(1, -1) if per_tensor else x
        amax = xs.abs().amax(dim=-1, keepdim=True)
        kt = (torch.frexp(amax).exponent - ebias).to(torch.int32)
        kt = torch.where(amax > 0, kt, torch.zeros_like(kt))
        assert torch.equal(k.reshape(-1), kt.reshape(-1))
        qt = (xs * torch.exp2((-kt).to(xs.dtype))).to(dt)
        assert torch.equal(q.reshape(-1).view(torch.uint8), qt.reshape(-1).view(torch.uint8))
        del qt
        d = fp8.dequantize(q, k, torch.bfloat16)
        dt_ = q.reshape(xs.shape).to(torch.bfloat16) * torch.exp2(kt.to(torch.bfloat16))
        assert torch.equal(d.reshape(-1), dt_.reshape(-1))
        del q, d
