"""The bookkeeping of accumulate.OrderedAccumulator on the CPU with int64
count lanes (the one part dtype the fold adds on the host, as
runtime/pieces.py:206-214 does): prefix-ordered folding of out-of-order
parts, quarantine holding its index until release or reject, the deferred
last part and its merge, the reference's duplicate and incompleteness
refusals (runtime/accumulate.py:15-137), and the attributes the reference's
stage reads (runtime/stage.py:175-177)."""

from __future__ import annotations

import pytest
import torch


def _lane(v: int) -> torch.Tensor:
    return torch.full((3,), v, dtype=torch.int64)


def test_prefix_order_quarantine_and_reject():
    from elysium_wan_amd.accumulate import OrderedAccumulator

    acc = OrderedAccumulator([0, 1, 2])
    acc.add(2, [_lane(200), _lane(201)])
    assert acc.pos == 0 and not acc.complete()
    acc.add(1, [_lane(100), _lane(101)], verified=False)
    acc.add(0, [_lane(1), _lane(2)])
    assert acc.pos == 1  # mb 1 is quarantined: the fold stops there
    acc.reject(1, [_lane(10), _lane(20)])
    assert acc.complete() and acc.pos == 3
    s = acc.result()
    assert torch.equal(s[0], _lane(211)) and torch.equal(s[1], _lane(223))
    with pytest.raises(AssertionError, match="duplicate"):
        acc.add(0, [_lane(0), _lane(0)])
    with pytest.raises(AssertionError, match="not quarantined"):
        acc.release(2)


def test_fold_part_holds_only_the_tensor_whose_prefix_is_missing():
    from elysium_wan_amd.accumulate import OrderedAccumulator

    acc = OrderedAccumulator(range(2))
    acc.fold_part(1, 0, 2, _lane(5))
    acc.fold_part(0, 1, 2, _lane(7))
    assert list(acc.next) == [0, 1] and (1, 0) in acc.parts and len(acc.parts) == 1
    acc.fold_part(0, 0, 2, _lane(1))
    assert list(acc.next) == [2, 1] and (1, 0) not in acc.parts
    acc.end_part(0)
    with pytest.raises(AssertionError, match="incomplete"):
        acc.result()
    acc.fold_part(1, 1, 2, _lane(3))
    acc.end_part(1)
    assert [int(t[0]) for t in acc.result()] == [6, 10]
    with pytest.raises(AssertionError, match="duplicate"):
        acc.fold_part(1, 0, 2, _lane(5))


@pytest.mark.parametrize("m", [1, 3])
def test_deferred_last_part_and_its_merge(m):
    from elysium_wan_amd.accumulate import OrderedAccumulator

    acc = OrderedAccumulator(range(m), defer_last=True)
    for mb in reversed(range(m)):
        acc.add(mb, [_lane(10**mb), _lane(2 * 10**mb)])
    assert acc.complete()
    grads, accs = acc.step_inputs()
    assert [int(g[0]) for g in grads] == [10 ** (m - 1), 2 * 10 ** (m - 1)]
    if m == 1:
        assert accs is None
    else:
        assert [int(a[0]) for a in accs] == [sum(10**k for k in range(m - 1)), 2 * sum(10**k for k in range(m - 1))]
    total = acc.result()
    assert [int(t[0]) for t in total] == [sum(10**k for k in range(m)), 2 * sum(10**k for k in range(m))]
    with pytest.raises(ValueError, match="already folded"):
        acc.step_inputs()
    with pytest.raises(ValueError, match="defer_last"):
        OrderedAccumulator([0]).step_inputs()


def test_stage_reads_order_next_and_parts_as_the_reference_does():
    """runtime/stage.py:175-177 asks, per tensor, whether microbatch mb's part
    is neither held nor already folded: `(mb, i) not in a.parts and
    a.next[i] <= k`; `a.next` is None before any part."""
    from elysium_wan_amd.accumulate import OrderedAccumulator

    acc = OrderedAccumulator([5, 3, 9])
    assert acc.next is None and len(acc.parts) == 0 and acc.pos == 0
    acc.fold_part(3, 0, 2, _lane(1))  # held: mb 5 is missing
    k = acc.order.index(3)
    missing = [i for i in range(2) if (3, i) not in acc.parts and acc.next[i] <= k]
    assert missing == [1]
    acc.fold_part(5, 0, 2, _lane(2))
    acc.fold_part(5, 1, 2, _lane(3))
    acc.end_part(5)
    assert list(acc.next) == [2, 1] and acc.closed == {5} and acc.added == 1
    acc.add(9, [_lane(4), _lane(5)], verified=False)
    assert acc.quarantine == {9} and (9, 0) in acc.parts
    acc.fold_part(3, 1, 2, _lane(6))
    acc.end_part(3)
    assert list(acc.next) == [2, 2] and not acc.complete()
    acc.release(9)
    assert acc.complete() and [int(t[0]) for t in acc.result()] == [7, 14]


def test_microbatch_outside_the_order_is_held_and_never_folded():
    from elysium_wan_amd.accumulate import OrderedAccumulator

    acc = OrderedAccumulator([0])
    acc.add(7, [_lane(1)])
    assert (7, 0) in acc.parts and acc.pos == 0 and not acc.complete()
    acc.add(0, [_lane(2)])
    # the reference counts every closed microbatch: two closed for an order of one
    assert not acc.complete()
    with pytest.raises(AssertionError, match="incomplete: 2/1 microbatches in, 1 tensors held"):
        acc.result()
