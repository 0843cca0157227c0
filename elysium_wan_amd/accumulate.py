"""The fixed-order gradient folds in front of the optimizer on MI355X: the
drop-in for wantrain's runtime/accumulate.py (OrderedAccumulator :15-137,
TiedRowFold :140-247).  The host-only MoE count fold (CountFold :250-318)
has no GPU work and stays the reference's own.

The step gradient is the iterative sum g_0 + g_1 + ... + g_{M-1} in
microbatch order, per tensor: the first part copied (widened to the sum's
dtype when a part comes narrower), then one add per later part.  Parts may
arrive in any order; each tensor folds as far as its prefix is complete and
holds what arrives early, so the sums equal the whole-set fold bit for bit.
A quarantined microbatch keeps its place in the order and blocks the fold
there until it is released or replaced.

Sums are fp32 on the GPU (the fp32 masters' gradients, with bf16 or fp32
parts): the adds run through pieces.fold_add's kernel (acc + widen(g), one
fp32 rounding).  A bf16 sum (bf16 parts with no wider dtype asked for)
folds through ely_fold_add_bf16, the fp32 add rounded to bf16 as torch's
add_ does.  int64 count lanes fold by torch's exact integer add, as
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

import numpy as np
import torch

from . import _lib, pieces


class _Inbox:
    """The parts handed in and not folded yet, as `acc.parts` shows them to
    a caller: `(mb, i) in acc.parts` and `len(acc.parts)`.  The reference's
    stage reads exactly that (runtime/stage.py:175-177)."""

    def __init__(self, owner: "OrderedAccumulator") -> None:
        self._owner = owner

    def __contains__(self, key) -> bool:
        mb, i = key
        return i in self._owner._box(mb)

    def __len__(self) -> int:
        o = self._owner
        return sum(len(b) for b in o._slots) + sum(len(b) for b in o._stray.values())


class OrderedAccumulator:
    """The step gradient's fixed-order fold (runtime/accumulate.py:15-137;
    the same methods, arguments and refusals).

    Bookkeeping: every microbatch of `order` has a position k.  Arrivals go
    to the inbox of their position (a dict of tensor index -> part), a
    quarantine mark and a closed mark are flags of the position, and
    `next[i]` (a numpy array) is the position tensor i folds next.  Tensor
    i advances while the inbox at its cursor holds its part and that
    position is not quarantined.  Microbatch ids outside `order` are kept
    apart and never folded, so the fold cannot complete with them missing.
    """

    def __init__(self, order, defer_last: bool = False):
        self.order = list(order)
        self._pos_of = {mb: k for k, mb in enumerate(self.order)}
        m = len(self.order)
        self._slots = [dict() for _ in range(m)]  # position -> {tensor index: part}
        self._held = np.zeros(m, dtype=bool)  # position in quarantine
        self._in = np.zeros(m, dtype=bool)  # position closed (every tensor handed in)
        self._stray: dict = {}  # microbatch id outside `order` -> {tensor index: part}
        self._stray_flags: dict = {}  # ... -> [quarantined, closed]
        self.parts = _Inbox(self)
        self.acc = None  # the sums, one per tensor index, once the tensor count is known
        self.next = None  # numpy int64 cursors, one per tensor index
        self.widen: dict = {}  # tensor index -> dtype of its sum (fold_part's dtype)
        self.defer_last = bool(defer_last)
        self.last = None  # defer_last: the held part of order[-1], per tensor index
        self._merged = False

    # ---------------------------------------------------------------- state

    def _box(self, mb) -> dict:
        k = self._pos_of.get(mb)
        return self._slots[k] if k is not None else self._stray.get(mb, {})

    def _flags(self, mb):
        k = self._pos_of.get(mb)
        if k is not None:
            return bool(self._held[k]), bool(self._in[k])
        q, c = self._stray_flags.get(mb, (False, False))
        return q, c

    def _mark(self, mb, *, held=None, closed=None) -> None:
        k = self._pos_of.get(mb)
        if k is None:
            f = self._stray_flags.setdefault(mb, [False, False])
            if held is not None:
                f[0] = held
            if closed is not None:
                f[1] = closed
            return
        if held is not None:
            self._held[k] = held
        if closed is not None:
            self._in[k] = closed

    def _put(self, mb, i: int, t) -> None:
        k = self._pos_of.get(mb)
        (self._slots[k] if k is not None else self._stray.setdefault(mb, {}))[i] = t

    @property
    def quarantine(self) -> set:
        """Microbatch ids held for an auditor's verdict."""
        out = {self.order[k] for k in np.flatnonzero(self._held)}
        return out | {mb for mb, f in self._stray_flags.items() if f[0]}

    @property
    def closed(self) -> set:
        """Microbatch ids whose every tensor was handed in."""
        out = {self.order[k] for k in np.flatnonzero(self._in)}
        return out | {mb for mb, f in self._stray_flags.items() if f[1]}

    @property
    def added(self) -> int:
        return int(self._in.sum()) + sum(1 for f in self._stray_flags.values() if f[1])

    @property
    def pos(self) -> int:
        """Microbatches of `order` that every tensor has taken (folded, or
        held as the deferred last part)."""
        return int(self.next.min()) if self.next is not None and self.next.size else 0

    def _size(self, n: int) -> None:
        if self.acc is None:
            self.acc = [None] * n
            self.next = np.zeros(n, dtype=np.int64)
            self.last = [None] * n
        if len(self.acc) != n:
            raise AssertionError(f"{n} tensors where the fold holds {len(self.acc)}")

    # ---------------------------------------------------------------- input

    def add(self, mb, tensors, verified: bool = True) -> None:
        """A whole microbatch; verified=False quarantines it."""
        if self._flags(mb)[1]:
            raise AssertionError(f"duplicate contribution for mb {mb}")
        self._size(len(tensors))
        if not verified:
            self._mark(mb, held=True)
        box = self._box(mb)
        for i, t in enumerate(tensors):
            if i in box:
                raise AssertionError(f"duplicate contribution for mb {mb}")
            self._put(mb, i, t)
            box = self._box(mb)
        self._mark(mb, closed=True)
        self._advance_all()

    def fold_part(self, mb, i: int, n: int, g, dtype=None) -> None:
        """Tensor i of the n of microbatch mb: folded now when every earlier
        microbatch's tensor i is in, held otherwise.  `dtype`: the sum's
        dtype when g may come narrower (a held part stays narrow)."""
        if self._flags(mb)[1] or i in self._box(mb):
            raise AssertionError(f"duplicate contribution for mb {mb} tensor {i}")
        self._size(n)
        if dtype is not None:
            self.widen[i] = dtype
        self._put(mb, i, g)
        self._advance(i)

    def end_part(self, mb) -> None:
        """Closes microbatch mb once all of its tensors went through fold_part."""
        if self._flags(mb)[1]:
            raise AssertionError(f"duplicate contribution for mb {mb}")
        self._size(0 if self.acc is None else len(self.acc))
        self._mark(mb, closed=True)

    def release(self, mb) -> None:
        """An auditor's verdict that the held microbatch is honest."""
        if not self._flags(mb)[0]:
            raise AssertionError(f"mb {mb} is not quarantined")
        self._mark(mb, held=False)
        self._advance_all()

    def reject(self, mb, replacement) -> None:
        """An auditor's recompute replaces the held microbatch's tensors."""
        if not self._flags(mb)[0]:
            raise AssertionError(f"mb {mb} is not quarantined")
        for i, t in enumerate(replacement):
            self._put(mb, i, t)
        self._mark(mb, held=False)
        self._advance_all()

    # ----------------------------------------------------------------- fold

    def _advance(self, i: int) -> None:
        """Tensor i takes every part from its cursor on that is in and not
        quarantined, in position order."""
        end = len(self.order)
        k = int(self.next[i])
        while k < end and not self._held[k]:
            t = self._slots[k].pop(i, None)
            if t is None:
                break
            self._take(i, k, t)
            k += 1
        self.next[i] = k

    def _advance_all(self) -> None:
        for i in range(len(self.acc)):
            self._advance(i)

    def _take(self, i: int, k: int, t) -> None:
        if self.defer_last and k == len(self.order) - 1:
            # folded inside the update (FusedAdamW.step(acc=...)) or by result()
            self.last[i] = t
        elif k == 0:
            self.acc[i] = self._first(i, t)
        else:
            pieces.fold_add(self.acc[i], t)

    def _first(self, i: int, t):
        """The sum's first value: a copy of the part, widened exactly when the
        sum is kept wider (bf16 to fp32 by pieces.fold_start's kernel)."""
        want = self.widen.get(i)
        if want is None or t.dtype == want:
            return t.clone()
        if want == torch.float32 and t.dtype == torch.bfloat16 and t.is_cuda:
            return pieces.fold_start(t)
        return t.to(want, copy=True)

    # --------------------------------------------------------------- output

    def complete(self) -> bool:
        end = len(self.order)
        return (self.added == end and self.acc is not None
                and bool(np.all(self.next == end)))

    def _check_complete(self) -> None:
        if not self.complete():
            raise AssertionError(
                f"accumulator incomplete: {self.added}/{len(self.order)} microbatches in, "
                f"{len(self.parts)} tensors held ({len(self.quarantine)} in quarantine)"
            )

    def result(self):
        """The sums, one per tensor (under defer_last the held last parts are
        folded in first)."""
        self._check_complete()
        if self.defer_last and not self._merged:
            for i, t in enumerate(self.last):
                if len(self.order) == 1:
                    self.acc[i] = self._first(i, t)
                else:
                    pieces.fold_add(self.acc[i], t)
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


class _HeldRows:
    """One microbatch's Head rows that an earlier microbatch still holds (or
    that its own embedding rows touch), waiting for its embedding rows."""

    __slots__ = ("k", "rows_host", "rows_dev", "h_rows", "ids", "first", "places_dev")

    def __init__(self, k, rows_host, rows_dev, h_rows, ids, first, places_dev):
        self.k = k  # the microbatch's position in the order
        self.rows_host = rows_host  # held row ids (numpy int64, ascending)
        self.rows_dev = rows_dev  # the same on the GPU
        self.h_rows = h_rows  # the Head gradient on those rows (a copy)
        self.ids = ids  # T_mb, the microbatch's own row ids (numpy)
        self.first = first  # the microbatch assigns rather than adds
        self.places_dev = places_dev  # each held row's place in T_mb, -1 if untouched (GPU)


class TiedRowFold:
    """The tied table's row fold on the Head (runtime/accumulate.py:140-247;
    the same methods, arguments and refusals): the step gradient
    acc = g_0, acc = acc + g_i in microbatch order with g_i = h_i + e_i
    (e_i = +0.0 outside the microbatch's rows T_i), bit for bit, without a
    dense table per microbatch in flight.

    add_head(mb, h, rows): h the (n_rows, d) gradient of the Head's use (fp32
    or bf16, on the GPU; every microbatch's of one shape, dtype and device),
    rows T_mb (ascending unique ids, int64).  add_embed(mb, e_rows):
    e_mb[T_mb] in ascending id.  Either may come first, for any microbatch
    of the order; an id outside the order is refused with a RuntimeError
    (the reference would hold it forever without folding it).

    Bookkeeping: each microbatch of the order has a position with a state
    (no Head gradient taken / rows held / done) and slots for what has
    arrived.  Head gradients are taken in position order.  Taking one folds
    its free rows at once, h + 0.0 (ely_rows_split, one launch), and keeps
    a copy of the rest: the rows an earlier microbatch still holds (a count
    per row) and its own T_mb.  The queue of held microbatches resolves
    front first once each one's embedding rows are in, as h + e on the held
    rows (ely_rows_fold, reading the embedding rows in place).  Every row
    therefore sees the stock sequence of adds."""

    _WAIT, _HELD, _DONE = 0, 1, 2

    def __init__(self, n_rows: int, order) -> None:
        self.n_rows = int(n_rows)
        if not 0 <= self.n_rows < 2**31:
            raise ValueError(f"tied fold: a table of {self.n_rows} rows (the row slots are int32)")
        self.order = list(order)
        self._k = {mb: k for k, mb in enumerate(self.order)}
        m = len(self.order)
        self._state = np.zeros(m, dtype=np.int8)
        self._head_at: list = [None] * m  # position -> (h, T_mb) until taken
        self._embed_at: list = [None] * m  # position -> e rows until resolved
        self._queue: list = []  # _HeldRows, oldest position first
        self._taken = 0  # Head gradients taken (positions 0 .. _taken-1)
        self._holds = np.zeros(self.n_rows, dtype=np.int32)  # per row: held microbatches
        self._like = None  # (d, dtype, device) every Head gradient shares
        self.acc = torch.empty(0)  # allocated by the first Head gradient taken

    @property
    def pos(self) -> int:
        """Head gradients taken so far, in order."""
        return self._taken

    def _position(self, mb, what: str) -> int:
        k = self._k.get(mb)
        if k is None:
            raise RuntimeError(f"tied fold: {what} for microbatch {mb}, which is not in the fold order")
        return k

    # ---------------------------------------------------------------- input

    def add_head(self, mb: int, h: torch.Tensor, rows: torch.Tensor) -> None:
        k = self._position(mb, "a Head gradient")
        if self._head_at[k] is not None or self._state[k] != self._WAIT:
            raise RuntimeError(f"tied fold: a second Head gradient for microbatch {mb}")
        if h.dim() != 2 or h.shape[0] != self.n_rows:
            raise RuntimeError(f"tied fold: Head gradient of mb {mb} has shape {tuple(h.shape)}")
        _lib.require_gpu(h, "tied fold")
        _lib.dtype_code(h)
        like = (int(h.shape[1]), h.dtype, h.device)
        if self._like is None:
            self._like = like
        elif like != self._like:
            # the kernels size rows from the first gradient's width and dtype
            raise RuntimeError(
                f"tied fold: Head gradient of mb {mb} is ({h.shape[1]} wide, {h.dtype}, {h.device}); "
                f"the fold holds ({self._like[0]} wide, {self._like[1]}, {self._like[2]})"
            )
        ids = np.ascontiguousarray(rows.to(torch.int64).cpu().numpy())
        self._head_at[k] = (h.contiguous(), ids)
        self._pump()

    def add_embed(self, mb: int, e_rows: torch.Tensor) -> None:
        k = self._position(mb, "an embedding gradient")
        if self._embed_at[k] is not None or self._state[k] == self._DONE:
            raise RuntimeError(f"tied fold: a second embedding gradient for microbatch {mb}")
        self._embed_at[k] = e_rows
        self._pump()

    def _pump(self) -> None:
        """Resolve the oldest held microbatch while its embedding rows are in;
        take the next Head gradient in order while it is in."""
        while True:
            if self._queue and self._embed_at[self._queue[0].k] is not None:
                self._resolve(self._queue.pop(0))
            elif self._taken < len(self.order) and self._head_at[self._taken] is not None:
                self._take(self._taken)
            else:
                return

    # ----------------------------------------------------------------- fold

    def _take(self, k: int) -> None:
        h, ids = self._head_at[k]
        self._head_at[k] = None
        first = self._taken == 0
        n = self.n_rows
        if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= n):
            raise RuntimeError(f"tied fold: rows of mb {self.order[k]} outside [0, {n})")
        if first:
            self.acc = torch.empty_like(h)
        held = self._holds > 0
        held[ids] = True
        rows = np.flatnonzero(held)
        nh = rows.size
        place = np.full(n, -1, dtype=np.int64)
        place[ids] = np.arange(ids.size, dtype=np.int64)
        # one pinned block up per Head gradient: the held rows, their places
        # in T_mb, and every row's slot among the held ones (-1: free); torch's
        # pinned-memory cache keeps it until the copy on this stream is done
        blk = torch.empty(2 * nh + (n + 1) // 2, dtype=torch.int64, pin_memory=True)
        b = blk.numpy()
        b[:nh] = rows
        b[nh:2 * nh] = place[rows]
        slot = b[2 * nh:].view(np.int32)[:n]
        slot.fill(-1)
        slot[rows] = np.arange(nh, dtype=np.int32)
        dev = h.device
        up = blk.to(dev, non_blocking=True)
        rows_d, places_d, slot_d = up[:nh], up[nh:2 * nh], up[2 * nh:].view(torch.int32)
        # free rows folded (acc = h + 0.0, or acc + (h + 0.0)); held rows
        # copied out of h bit for bit, so h itself need not be kept
        h_rows = torch.empty((nh, h.shape[1]), dtype=h.dtype, device=dev)
        L = _lib.load()
        _lib.check(L.ely_rows_split(self.acc.data_ptr(), h.data_ptr(), slot_d.data_ptr(), h_rows.data_ptr() if nh else None,
                                    n, nh, h.shape[1], _lib.dtype_code(self.acc), int(first), _lib.stream_ptr(dev)),
                   "tied fold")
        self._queue.append(_HeldRows(k, rows, rows_d, h_rows, ids, first, places_d))
        self._holds[rows] += 1
        self._state[k] = self._HELD
        self._taken += 1

    def _resolve(self, r: _HeldRows) -> None:
        e_rows = self._embed_at[r.k]
        self._embed_at[r.k] = None
        mb = self.order[r.k]
        d = r.h_rows.shape[1]
        if e_rows.dim() != 2 or e_rows.shape[0] != r.ids.size or e_rows.shape[1] != d:
            raise RuntimeError(
                f"tied fold: embedding rows of mb {mb} have shape {tuple(e_rows.shape)}, "
                f"want ({r.ids.size}, {tuple(r.h_rows.shape[1:])})"
            )
        nh = r.rows_host.size
        if nh:
            e = e_rows.to(r.h_rows.device, r.h_rows.dtype).contiguous() if r.ids.size else None
            # held rows: acc = h + e_on (first) or acc + (h + e_on), e_on = e
            # at the row's place in T_mb and +0.0 where it has none
            L = _lib.load()
            _lib.check(L.ely_rows_fold(self.acc.data_ptr(), r.h_rows.data_ptr(), None,
                                       None if e is None else e.data_ptr(), None if e is None else r.places_dev.data_ptr(),
                                       r.rows_dev.data_ptr(), nh, self.n_rows, nh, 0 if e is None else e.shape[0],
                                       d, _lib.dtype_code(self.acc), int(r.first), _lib.stream_ptr(r.h_rows.device)),
                       "tied fold")
        self._holds[r.rows_host] -= 1
        self._state[r.k] = self._DONE

    # --------------------------------------------------------------- output

    def complete(self) -> bool:
        return self._taken == len(self.order) and not self._queue

    def result(self) -> torch.Tensor:
        if not self.complete():
            raise RuntimeError(
                f"tied fold incomplete: {self._taken}/{len(self.order)} Head gradients, "
                f"{len(self._queue)} microbatch(es) waiting for embedding rows"
            )
        return self.acc
