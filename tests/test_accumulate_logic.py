"""The bookkeeping of accumulate.OrderedAccumulator on the CPU with int64
count lanes (the one part dtype the fold adds on the host, as
runtime/pieces.py:206-214 does): prefix-ordered folding of out-of-order
parts, quarantine holding its index until release or reject, the deferred
last part and its merge, and the reference's duplicate and incompleteness
refusals (runtime/accumulate.py:15-137)."""

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
    assert acc.next == [0, 1] and (1, 0) in acc.parts
    acc.fold_part(0, 0, 2, _lane(1))
    assert acc.next == [2, 1]
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


def test_count_fold_sums_in_order_and_refuses_as_the_reference():
    """runtime/accumulate.py:250-318 on the host: int64 (E,) vectors per
    (microbatch, layer), summed exactly; the reference's refusals."""
    from elysium_wan_amd.accumulate import CountFold

    cf = CountFold(step=7, n_mb=2, layers=[3], experts={3: 4}, total={3: 6})
    cf.add(1, 3, torch.tensor([1, 2, 3, 0]), peer=1)
    assert not cf.complete() and cf.missing() == [(0, 3)]
    with pytest.raises(RuntimeError, match=r"MOE-COUNT \(step 7, mb 0, layer 3, peer -\): count vector missing at the owner \(1 missing\)"):
        cf.result()
    cf.add(0, 3, torch.tensor([0, 0, 6, 0]), peer=0)
    assert torch.equal(cf.result()[3], torch.tensor([1, 2, 9, 0]))
    bad = [
        ((2, 3, torch.zeros(4, dtype=torch.int64)), "microbatch outside"),
        ((0, 9, torch.zeros(4, dtype=torch.int64)), "no selection bias"),
        ((0, 3, torch.zeros(4, dtype=torch.int64)), "given twice"),
    ]
    for args, msg in bad:
        with pytest.raises(RuntimeError, match=msg):
            cf.add(*args, peer=2)
    fresh = CountFold(step=1, n_mb=1, layers=[0], experts={0: 2}, total={0: 3})
    for vec, msg in ((torch.zeros(2), "not an int64"), (torch.zeros(3, dtype=torch.int64), "shape"),
                     (torch.tensor([-1, 4]), "negative"), (torch.tensor([1, 1]), "sum to 2, want T_mb\\*k = 3")):
        with pytest.raises(RuntimeError, match=msg):
            fresh.add(0, 0, vec, peer=0)
