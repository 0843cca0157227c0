"""The tied table's row fold (accumulate.TiedRowFold, the drop-in for
runtime/accumulate.py:140-247) on the GPU: Head gradients and embedding rows
handed in out of order, rows held by earlier microbatches, fp32 and bf16
tables, aligned and unaligned rows -- the result equals the stock fold
acc = g_0, acc = acc + g_i (g_i = h_i + e_i, e_i = +0 outside the
microbatch's rows, each add rounded to the table's dtype) computed on the
CPU, bit for bit, including the +0.0 that h + 0.0 makes of a -0.0."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from gpu_util import bits, say

pytestmark = pytest.mark.gpu


def _stock_fold(oracle, hs, rows, es, dtype):
    """The reference's dense fold in microbatch order (numpy, IEEE fp32 adds,
    bf16 rounding by the oracle's RNE after each add for bf16 tables)."""
    acc = None
    for h, r, e in zip(hs, rows, es):
        hf = bits(h.float()).astype(np.float32)
        E = np.zeros_like(hf)  # +0.0 outside the microbatch's rows
        E[r.numpy()] = bits(e.float())
        g = hf + E
        if dtype == torch.bfloat16:
            g = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(g)).reshape(hf.shape)
        if acc is None:
            acc = g
        else:
            acc = acc + g
            if dtype == torch.bfloat16:
                acc = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(acc)).reshape(hf.shape)
    return acc


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 37])
def test_out_of_order_heads_and_embeddings_equal_the_stock_fold(oracle, dtype, d):
    from elysium_wan_amd.accumulate import TiedRowFold

    n_rows, M = 1000, 5
    gen = torch.Generator().manual_seed(90 + d)
    hs, rows, es = [], [], []
    for mb in range(M):
        h = torch.randn(n_rows, d, generator=gen)
        h[torch.rand(n_rows, d, generator=gen) < 0.01] = -0.0  # h + 0.0 turns these into +0.0
        r = torch.randperm(n_rows, generator=gen)[: 40 + 30 * mb].sort().values
        hs.append(h.to(dtype))
        rows.append(r)
        es.append(torch.randn(r.numel(), d, generator=gen).to(dtype))
    fold = TiedRowFold(n_rows, range(M))
    say("tied fold", dtype, d)
    # Head gradients and embedding rows arrive out of order and interleaved
    events = [("h", 2), ("e", 1), ("h", 0), ("e", 3), ("h", 1), ("e", 0), ("h", 4), ("h", 3), ("e", 4), ("e", 2)]
    for kind, mb in events:
        if kind == "h":
            fold.add_head(mb, hs[mb].cuda(), rows[mb])
        else:
            fold.add_embed(mb, es[mb].cuda())
    assert fold.complete()
    got = fold.result()
    torch.cuda.synchronize()
    want = _stock_fold(oracle, hs, rows, es, dtype)
    gotf = bits(got.float()).astype(np.float32).reshape(-1)
    assert np.array_equal(gotf.view(np.uint32), want.reshape(-1).view(np.uint32))
    with pytest.raises(RuntimeError, match="second Head"):
        fold.add_head(0, hs[0].cuda(), rows[0])


def test_incomplete_fold_names_what_it_waits_for():
    from elysium_wan_amd.accumulate import TiedRowFold

    fold = TiedRowFold(8, range(2))
    fold.add_head(0, torch.randn(8, 4, device="cuda"), torch.tensor([1, 5]))
    with pytest.raises(RuntimeError, match="tied fold incomplete: 1/2 Head gradients, 1 microbatch"):
        fold.result()
    with pytest.raises(RuntimeError, match="embedding rows of mb 0 have shape"):
        fold.add_embed(0, torch.randn(3, 4, device="cuda"))


def test_a_head_gradient_unlike_the_first_is_refused_before_any_launch():
    """The row kernels size every row from the fold's table: a later Head
    gradient of another width, dtype or device is refused at add_head, as
    the reference's own shape and dtype errors stop it, and nothing of it
    reaches the GPU; the fold then finishes as if it never came."""
    from elysium_wan_amd.accumulate import TiedRowFold

    fold = TiedRowFold(8, range(2))
    h0 = torch.randn(8, 4, device="cuda")
    fold.add_head(1, h0, torch.tensor([2]))  # held: microbatch 0 comes later
    for bad in (torch.randn(8, 5, device="cuda"), torch.randn(8, 4, device="cuda").to(torch.bfloat16),
                torch.randn(8, 4, dtype=torch.float64, device="cuda")):
        with pytest.raises((RuntimeError, TypeError)):
            fold.add_head(0, bad, torch.tensor([1]))
    with pytest.raises(RuntimeError, match="not in the fold order"):
        fold.add_head(7, h0, torch.tensor([1]))
    h1 = torch.randn(8, 4, device="cuda")
    fold.add_head(0, h1, torch.tensor([1]))
    e0, e1 = torch.randn(1, 4, device="cuda"), torch.randn(1, 4, device="cuda")
    fold.add_embed(0, e0)
    fold.add_embed(1, e1)
    assert fold.complete()
    # the stock fold: g_i = h_i + E_i (E_i zero outside T_i), acc = g_0 + g_1
    E0, E1 = torch.zeros_like(h1), torch.zeros_like(h0)
    E0[1], E1[2] = e0[0], e1[0]
    stock = (h1 + E0) + (h0 + E1)
    torch.cuda.synchronize()
    assert torch.equal(fold.result().view(torch.int32), stock.view(torch.int32))


@settings(max_examples=25, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
@given(
    m=st.integers(1, 5),
    n_rows=st.sampled_from([1, 7, 64, 333]),
    d=st.sampled_from([1, 8, 24, 40]),
    bf16=st.booleans(),
    perm_seed=st.integers(0, 2**16),
    data_seed=st.integers(0, 2**16),
)
def test_tied_fold_fuzz_equals_the_stock_fold(oracle, m, n_rows, d, bf16, perm_seed, data_seed):
    """Random microbatch counts, table shapes (rows that fit a vector and rows
    that do not), row sets (empty and full included) and arrival orders of
    the 2M events: the GPU fold equals the CPU stock fold bit for bit."""
    import random

    from elysium_wan_amd.accumulate import TiedRowFold

    dtype = torch.bfloat16 if bf16 else torch.float32
    gen = torch.Generator().manual_seed(data_seed)
    hs, rows, es = [], [], []
    for mb in range(m):
        h = torch.randn(n_rows, d, generator=gen)
        h[torch.rand(n_rows, d, generator=gen) < 0.05] = -0.0
        k = int(torch.randint(0, n_rows + 1, (1,), generator=gen))
        r = torch.randperm(n_rows, generator=gen)[:k].sort().values
        hs.append(h.to(dtype))
        rows.append(r)
        es.append(torch.randn(k, d, generator=gen).to(dtype))
    events = [("h", mb) for mb in range(m)] + [("e", mb) for mb in range(m)]
    random.Random(perm_seed).shuffle(events)
    say("tied fold fuzz", m, n_rows, d, dtype, events)
    fold = TiedRowFold(n_rows, range(m))
    for kind, mb in events:
        if kind == "h":
            fold.add_head(mb, hs[mb].cuda(), rows[mb])
        else:
            fold.add_embed(mb, es[mb].cuda())
    assert fold.complete()
    got = bits(fold.result().float()).astype(np.float32).reshape(-1)
    torch.cuda.synchronize()
    want = _stock_fold(oracle, hs, rows, es, dtype).reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_tied_fold_at_the_benchmark_size_equals_the_dense_fold(dtype):
    """The tied_fold leg's shape: a 32,768 x 2,560 table, 8 microbatches of
    4,096 rows, the embedding rows one microbatch behind the Head gradients
    (the held set grows to the union of the rows seen): the result equals
    the reference's dense fold in torch ops (e scattered into a zero table,
    g = h + e, acc = g_0 then acc += g_i, runtime/accumulate.py:145-160)
    bit for bit."""
    from elysium_wan_amd.accumulate import TiedRowFold

    n_mb, n_rows, d, k = 8, 32768, 2560, 4096
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(23)
    hs = [(torch.randn(n_rows, d, device=dev, generator=gen) * 1e-3).to(dtype) for _ in range(n_mb)]
    rows = [torch.randperm(n_rows, device=dev, generator=gen)[:k].sort().values.cpu() for _ in range(n_mb)]
    es = [(torch.randn(k, d, device=dev, generator=gen) * 1e-3).to(dtype) for _ in range(n_mb)]
    say("tied fold at the benchmark size", dtype)
    fold = TiedRowFold(n_rows, range(n_mb))
    for mb in range(n_mb):
        fold.add_head(mb, hs[mb], rows[mb])
        if mb:
            fold.add_embed(mb - 1, es[mb - 1])
    fold.add_embed(n_mb - 1, es[n_mb - 1])
    got = fold.result()
    acc = None
    for mb in range(n_mb):
        e = torch.zeros(n_rows, d, device=dev, dtype=dtype)
        e[rows[mb].to(dev)] = es[mb]
        g = hs[mb] + e
        acc = g if acc is None else acc.add_(g)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       acc.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
