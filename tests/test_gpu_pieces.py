"""The pieces kernels on the GPU: the fp32 -> bf16 working-copy cast bit for
bit against torch-on-GPU's `.to(bfloat16)` (NaN, Inf, ties, subnormals
included) and the oracle, and the ordered fp32 fold (runtime/pieces.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import bits, say

pytestmark = pytest.mark.gpu


def test_cast_piece_equals_torch_on_the_gpu(oracle):
    from elysium_wan_amd import pieces

    g = torch.Generator().manual_seed(0)
    u = torch.randint(-(1 << 31), 1 << 31, (3_000_001,), generator=g, dtype=torch.int64).to(torch.int32)
    ties = (torch.randint(0, 1 << 16, (10000,), generator=g, dtype=torch.int64) << 16 | 0x8000).to(torch.int32)
    x = torch.cat([u, ties]).view(torch.float32).cuda()
    for view in (x, x[1:]):  # aligned and 4 bytes off
        say("cast_piece", view.data_ptr() % 16)
        got = pieces.cast_piece(view, torch.bfloat16)
        assert got.data_ptr() != view.data_ptr()
        assert np.array_equal(bits(got), bits(view.to(torch.bfloat16)))
        assert np.array_equal(bits(got), oracle.f32_to_bf16_bits(bits(view)))


def test_fold_is_widen_then_add_in_order(oracle):
    from elysium_wan_amd import pieces

    gen = torch.Generator().manual_seed(1)
    parts = [torch.randn(100003, generator=gen).bfloat16() for _ in range(3)] + [torch.randn(100003, generator=gen)]
    say("fold")
    acc = pieces.fold([p.cuda() for p in parts])
    ref = parts[0].float().numpy().copy()
    for p in parts[1:]:
        oracle.fold_add(ref, bits(p) if p.dtype == torch.bfloat16 else p.numpy())
    assert np.array_equal(bits(acc).view(np.uint32), ref.view(np.uint32))
    # tests/unit/test_stream_fold.py:213-236: a bf16 part folded into an fp32
    # sum equals widen-then-add
    a = torch.randn(5000, device="cuda")
    b = torch.randn(5000, device="cuda").bfloat16()
    want = a + b.float()
    pieces.fold_add(a, b)
    assert torch.equal(a, want)


def test_step_unit_steps_only_its_unit():
    """runtime/pieces.py:235-256 with pieces.adamw (torch's AdamW op order):
    the unit's params move exactly as a whole-list step over them would;
    the other unit's params, moments and step counters stay untouched."""
    from elysium_wan_amd import pieces

    gen = torch.Generator().manual_seed(11)
    shapes = [(64, 48), (48,), (300,), (17, 5)]
    init = [torch.randn(s, generator=gen) for s in shapes]
    ps = [t.clone().cuda().requires_grad_(True) for t in init]
    solo = [t.clone().cuda().requires_grad_(True) for t in init[:2]]
    opt = pieces.adamw(ps, 1e-2)
    opt_solo = pieces.adamw(solo, 1e-2)
    say("step_unit")
    for step in range(3):
        gs = [(torch.randn(s, generator=gen) * 1e-2).cuda() for s in shapes[:2]]
        pieces.step_unit(opt, ps[:2], gs)
        pieces.step_unit(opt_solo, solo, [g.clone() for g in gs])
    for a, b in zip(ps[:2], solo):
        assert torch.equal(a.detach().view(torch.int32), b.detach().view(torch.int32))
    for a, b in zip(ps[2:], init[2:]):
        assert torch.equal(a.detach().cpu(), b)
    # torch's AdamW keys its state by parameter (runtime/stage.py:2265-2271 reads it so)
    keys = list(opt.state)
    assert len(keys) == 2 and keys[0] is ps[0] and keys[1] is ps[1]
    assert all(float(opt.state[p]["step"]) == 3.0 for p in ps[:2])
    assert all(p.grad is None for p in ps)
    with pytest.raises(ValueError, match="outside"):
        pieces.step_unit(opt, [torch.zeros(3, device="cuda", requires_grad=True)], [torch.zeros(3, device="cuda")])


def test_elementwise_passes_over_several_grid_strides():
    """fold_add and the clip's in-place scale over 9M elements, several
    strides of every kernel's persistent grid, on aligned views and views one
    element off (the scalar path), bit for bit against torch on the GPU:
    a + widen(g) and g * coef are each one fp32 rounding (then one bf16
    rounding for a bf16 g)."""
    from elysium_wan_amd import _lib, pieces

    L = _lib.load()
    n = 9_000_003
    gen = torch.Generator(device="cuda").manual_seed(5)
    acc0 = torch.randn(n + 1, device="cuda", generator=gen)
    gf = torch.randn(n + 1, device="cuda", generator=gen)
    gb = torch.randn(n + 1, device="cuda", generator=gen).bfloat16()
    coef = torch.tensor([0.3712], device="cuda")
    for off in (0, 1):
        for g in (gb, gf):
            say("fold_add", g.dtype, "offset", off)
            a = acc0[off:].clone() if off == 0 else acc0.clone()[off:]
            want = a + g[off:].float()
            pieces.fold_add(a, g[off:])
            assert torch.equal(a, want)
            say("scale_inplace", g.dtype, "offset", off)
            h = g.clone()[off:]
            want = (h.float() * coef).to(g.dtype)
            _lib.check(L.ely_scale_inplace(_lib.tensor_array([h]), 1, coef.data_ptr(), _lib.stream_ptr(h.device)), "scale")
            assert torch.equal(bits_t(h), bits_t(want))


def bits_t(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)
