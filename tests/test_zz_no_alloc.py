"""ely_fp8_quantize_noalloc, the quantize entry point that allocates
nothing (its split path keeps row maxima in the library's static device
scratch), against ely_fp8_quantize with a caller workspace, through the C
ABI: codes and exponents byte for byte, two calls in a row with the second
smaller (the scratch keeps the first call's contents), on the split path
(per-tensor scaling, long rows, unaligned rows) and the register path, and
the refusal of a shape whose row maxima do not fit the scratch."""

from __future__ import annotations

import pytest
import torch

from gpu_util import say

pytestmark = pytest.mark.gpu


def _quantize_both(x: torch.Tensor, rows: int, cols: int, fmt: int):
    from elysium_wan_amd import _lib

    L = _lib.load()
    dt = _lib.dtype_code(x)
    s = _lib.stream_ptr(x.device)
    q0 = torch.empty(rows * cols, dtype=torch.uint8, device=x.device)
    k0 = torch.empty(max(rows, 1), dtype=torch.int32, device=x.device)
    ws = torch.empty(max(L.ely_fp8_workspace_bytes(rows, cols, dt), 256), dtype=torch.uint8, device=x.device)
    _lib.check(L.ely_fp8_quantize(x.data_ptr(), dt, rows, cols, fmt, q0.data_ptr(), k0.data_ptr(), ws.data_ptr(), ws.numel(), s),
               "ely_fp8_quantize")
    q1 = torch.full_like(q0, 0xA5)
    k1 = torch.full_like(k0, -999)
    _lib.check(L.ely_fp8_quantize_noalloc(x.data_ptr(), dt, rows, cols, fmt, q1.data_ptr(), k1.data_ptr(), s),
               "ely_fp8_quantize_noalloc")
    torch.cuda.synchronize()
    return (q0, k0[:rows]), (q1, k1[:rows])


# (rows, cols, dtype, offset): each pair is run larger first, then smaller
PAIRS = [
    ((100_000, 8200, torch.bfloat16, 0), (2, 50_000, torch.bfloat16, 0)),   # many split rows, then per-row split
    ((1, 1 << 24, torch.bfloat16, 0), (1, 1 << 20, torch.bfloat16, 0)),     # per-tensor scaling
    ((3, 1_000_003, torch.float32, 1), (1, 777_777, torch.bfloat16, 1)),    # unaligned: element path
    ((4096, 768, torch.bfloat16, 0), (16, 2560, torch.bfloat16, 0)),        # register path (no scratch)
]


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("pair", range(len(PAIRS)))
def test_noalloc_quantize_equals_the_workspace_entry_point(pair, fmt):
    gen = torch.Generator(device="cuda").manual_seed(100 + pair)
    for rows, cols, dtype, off in PAIRS[pair]:
        say("noalloc quantize", "e4m3" if fmt == 0 else "e5m2", rows, cols, dtype, "offset", off)
        buf = torch.empty(rows * cols + off, device="cuda", dtype=torch.float32).normal_(generator=gen)
        buf.view(-1)[:: max(1, rows * cols // 997)] *= 300.0
        x = buf.to(dtype)[off:]
        (q0, k0), (q1, k1) = _quantize_both(x, rows, cols, fmt)
        assert torch.equal(q0, q1)
        assert torch.equal(k0, k1)
        del buf, x, q0, q1, k0, k1
    torch.cuda.empty_cache()


def test_noalloc_quantize_refuses_more_rows_than_its_scratch_holds():
    from elysium_wan_amd import _lib

    L = _lib.load()
    rows, cols = 140_000, 8200  # split path: 2 x 560,000 bytes of row maxima > 1 MiB
    x = torch.zeros(rows * cols, dtype=torch.bfloat16, device="cuda")
    q = torch.empty(rows * cols, dtype=torch.uint8, device="cuda")
    k = torch.empty(rows, dtype=torch.int32, device="cuda")
    say("noalloc quantize refusal", rows, cols)
    rc = L.ely_fp8_quantize_noalloc(x.data_ptr(), _lib.BF16, rows, cols, 0, q.data_ptr(), k.data_ptr(), _lib.stream_ptr(x.device))
    assert rc == _lib.EINVAL
    assert "static scratch" in L.ely_last_error().decode()
    del x, q, k
    torch.cuda.empty_cache()
