"""Launches captured into a HIP graph (torch.cuda.graph) and replayed: the
no-allocation fp8 quantize on its split path (per-tensor scaling) and on its
register path, the grad-norm of a short list (its tables in the kernel
arguments) and the bf16 cast.  Before each replay new inputs are written
eagerly into the captured buffers, and every replay's outputs equal eager
calls on the same inputs, byte for byte."""

from __future__ import annotations

import pytest
import torch

from gpu_util import say

pytestmark = pytest.mark.gpu


def test_captured_launches_replay_like_eager_calls():
    from elysium_wan_amd import _lib

    L = _lib.load()
    dev = torch.device("cuda")
    x_t = torch.empty(1 << 22, dtype=torch.bfloat16, device=dev)  # one row: the split path
    x_r = torch.empty(512 * 2560, dtype=torch.bfloat16, device=dev)  # 512 rows of 2,560: registers
    q_t = torch.empty(x_t.numel(), dtype=torch.uint8, device=dev)
    k_t = torch.empty(1, dtype=torch.int32, device=dev)
    q_r = torch.empty(x_r.numel(), dtype=torch.uint8, device=dev)
    k_r = torch.empty(512, dtype=torch.int32, device=dev)
    gs = [torch.empty(n, dtype=torch.float32, device=dev) for n in (1000, 3 * 4096 + 5, 70_000)]
    garr = _lib.tensor_array(gs)
    res = torch.zeros(16, dtype=torch.uint8, device=dev)
    ws = torch.empty(max(L.ely_grad_norm_workspace_bytes(garr, len(gs)), 256), dtype=torch.uint8, device=dev)
    p = torch.empty(300_001, dtype=torch.float32, device=dev)
    c = torch.empty(p.numel(), dtype=torch.bfloat16, device=dev)
    outs = (q_t, k_t, q_r, k_r, res, c)

    def calls():
        s = _lib.stream_ptr(dev)  # the current stream: the capture stream while capturing
        _lib.check(L.ely_fp8_quantize_noalloc(x_t.data_ptr(), _lib.BF16, 1, x_t.numel(), 0, q_t.data_ptr(), k_t.data_ptr(), s),
                   "quantize per tensor")
        _lib.check(L.ely_fp8_quantize_noalloc(x_r.data_ptr(), _lib.BF16, 512, 2560, 1, q_r.data_ptr(), k_r.data_ptr(), s),
                   "quantize per row")
        _lib.check(L.ely_grad_norm(garr, len(gs), 1.0, res.data_ptr(), ws.data_ptr(), ws.numel(), s), "norm")
        _lib.check(L.ely_cast_bf16(p.data_ptr(), c.data_ptr(), p.numel(), s), "cast")

    def fill(seed):
        gen = torch.Generator(device=dev).manual_seed(seed)
        for t in (x_t, x_r):
            t.copy_(torch.randn(t.numel(), device=dev, generator=gen) * (10.0 ** (seed % 5 - 2)))
        for g in gs:
            g.normal_(generator=gen).mul_(1e-3 * (seed + 1))
        p.normal_(generator=gen)

    fill(0)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()  # warm-up off the default stream, as capture wants
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    say("capture: quantize x2, norm, cast")
    with torch.cuda.graph(graph):
        calls()
    for seed in (1, 2, 3, 4):
        fill(seed)
        graph.replay()
        torch.cuda.synchronize()
        replayed = [t.clone() for t in outs]
        for t in outs:
            t.fill_(0x5A if t.dtype == torch.uint8 else 7)  # eager results must not be the replay's leftovers
        calls()
        torch.cuda.synchronize()
        say("replay", seed)
        for a, b in zip(replayed, outs):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
