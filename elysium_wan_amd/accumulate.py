"""The fixed-order gradient fold in front of the optimizer on MI355X: the
drop-in for wantrain's runtime/accumulate.py:15-137 (OrderedAccumulator).

The step gradient is the iterative sum g_0 + g_1 + ... + g_{M-1} in
microbatch order, per tensor: the first part copied (widened to the sum's
dtype when a part comes narrower), then one add per later part.  Parts may
arrive in any order; each tensor folds as far as its prefix is complete and
holds what arrives early, so the sums equal the whole-set fold bit for bit.
A quarantined microbatch keeps its place in the order and blocks the fold
there until it is released or replaced.

Sums are fp32 on the GPU (the fp32 masters' gradients, with bf16 or fp32
parts): the adds run through pieces.fold_add's kernel (acc + widen(g), one
fp32 rounding).  int64 count lanes fold by torch's exact integer add, as
runtime/pieces.py:206-214 does.

defer_last=True (an addition to the reference's interface): each tensor's
part of the last microbatch in the order is held instead of folded.
step_inputs() then returns (grads, accs) for FusedAdamW.step(grads=grads,
acc=accs), which finishes the fold inside the update kernel
(ely_adamw_fold_step): the sum's 8-byte-per-element write-and-read pass is
never made, and the update's bits equal folding first.  result() still
returns the complete sums (folding the held parts then), so a caller that
needs them is unaffected.
"""

from __future__ import annotations

from . import pieces


class OrderedAccumulator:
    """runtime/accumulate.py:15-137: add(mb, tensors) hands in a whole
    microbatch; fold_part(mb, i, n, g, dtype) one tensor of it, end_part(mb)
    closes it; release / reject settle a quarantined microbatch; complete()
    and result() as the reference's."""

    def __init__(self, order, defer_last: bool = False):
        self.order = list(order)  # microbatch ids in fold order
        self.acc = None  # running sums, one per tensor index
        self.next = None  # per tensor index: position in `order` of its next fold
        self.parts: dict = {}  # (mb, i) -> part waiting for its prefix
        self.quarantine: set = set()
        self.closed: set = set()
        self.added = 0
        self.widen: dict = {}  # tensor index -> dtype its sum is kept in (fold_part's dtype)
        self.defer_last = bool(defer_last)
        self.last = None  # defer_last: per tensor index, the held part of order[-1]
        self._merged = False  # defer_last: result() folded the held parts in

    @property
    def pos(self) -> int:
        """Microbatches of `order` that every tensor has taken (folded, or
        held as the deferred last part)."""
        return min(self.next) if self.next else 0

    def _size(self, n: int) -> None:
        if self.acc is None:
            self.acc = [None] * n
            self.next = [0] * n
            self.last = [None] * n
        if len(self.acc) != n:
            raise AssertionError(f"{n} tensors where the fold holds {len(self.acc)}")

    def add(self, mb, tensors, verified: bool = True) -> None:
        if mb in self.closed:
            raise AssertionError(f"duplicate contribution for mb {mb}")
        self._size(len(tensors))
        if not verified:
            self.quarantine.add(mb)
        for i, t in enumerate(tensors):
            if (mb, i) in self.parts:
                raise AssertionError(f"duplicate contribution for mb {mb}")
            self.parts[(mb, i)] = t
        self.closed.add(mb)
        self.added += 1
        self._fold_all()

    def fold_part(self, mb, i: int, n: int, g, dtype=None) -> None:
        """Tensor i of the n of microbatch mb: folded now when every earlier
        microbatch's tensor i is in, held otherwise.  `dtype`: the sum's
        dtype when g may come narrower (a held part stays narrow)."""
        if mb in self.closed or (mb, i) in self.parts:
            raise AssertionError(f"duplicate contribution for mb {mb} tensor {i}")
        self._size(n)
        if dtype is not None:
            self.widen[i] = dtype
        self.parts[(mb, i)] = g
        self._fold(i)

    def end_part(self, mb) -> None:
        """Every tensor of microbatch mb was handed to fold_part."""
        if mb in self.closed:
            raise AssertionError(f"duplicate contribution for mb {mb}")
        self._size(0 if self.acc is None else len(self.acc))
        self.closed.add(mb)
        self.added += 1

    def _first(self, i: int, t):
        """The sum's first value: the part itself, copied (widened exactly
        when the sum is kept wider)."""
        want = self.widen.get(i)
        if want is not None and t.dtype != want:
            return t.to(want, copy=True)
        return t.clone()

    def _add(self, i: int, t) -> None:
        """acc[i] += t in place: fp32 sums on the GPU kernel, int64 count
        lanes by integer add (pieces.fold_add refuses other sums)."""
        pieces.fold_add(self.acc[i], t)

    def _fold(self, i: int) -> None:
        last = len(self.order) - 1
        while self.next[i] < len(self.order):
            nxt = self.order[self.next[i]]
            if nxt in self.quarantine or (nxt, i) not in self.parts:
                return
            t = self.parts.pop((nxt, i))
            if self.defer_last and self.next[i] == last:
                self.last[i] = t  # folded inside the update (FusedAdamW.step(acc=...)) or by result()
            elif self.next[i] == 0:
                self.acc[i] = self._first(i, t)
            else:
                self._add(i, t)
            self.next[i] += 1

    def _fold_all(self) -> None:
        for i in range(len(self.acc)):
            self._fold(i)

    def release(self, mb) -> None:
        """An auditor's verdict that the held microbatch is honest."""
        if mb not in self.quarantine:
            raise AssertionError(f"mb {mb} is not quarantined")
        self.quarantine.discard(mb)
        self._fold_all()

    def reject(self, mb, replacement) -> None:
        """An auditor's recompute replaces the held microbatch's tensors."""
        if mb not in self.quarantine:
            raise AssertionError(f"mb {mb} is not quarantined")
        for i, t in enumerate(replacement):
            self.parts[(mb, i)] = t
        self.quarantine.discard(mb)
        self._fold_all()

    def complete(self) -> bool:
        return len(self.closed) == len(self.order) and self.acc is not None and all(k == len(self.order) for k in self.next)

    def _check_complete(self) -> None:
        if not self.complete():
            raise AssertionError(
                f"accumulator incomplete: {len(self.closed)}/{len(self.order)} microbatches in, "
                f"{len(self.parts)} tensors held ({len(self.quarantine)} in quarantine)"
            )

    def result(self):
        """The sums, one per tensor (the held last parts folded in first
        under defer_last)."""
        self._check_complete()
        if self.defer_last and not self._merged:
            for i, t in enumerate(self.last):
                if len(self.order) == 1:
                    self.acc[i] = self._first(i, t)
                else:
                    self._add(i, t)
            self.last = [None] * len(self.acc)
            self._merged = True
        return self.acc

    def step_inputs(self):
        """defer_last: (grads, accs) for FusedAdamW.step(grads=..., acc=...):
        the held last parts and the sums of the microbatches before them
        (accs is None when the order holds one microbatch)."""
        if not self.defer_last:
            raise ValueError("step_inputs needs OrderedAccumulator(order, defer_last=True)")
        self._check_complete()
        if self._merged:
            raise ValueError("result() already folded the last parts in")
        return list(self.last), (None if len(self.order) == 1 else list(self.acc))
