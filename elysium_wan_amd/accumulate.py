"""The fixed-order gradient folds in front of the optimizer on MI355X: the
drop-in for wantrain's runtime/accumulate.py (OrderedAccumulator :15-137,
TiedRowFold :140-247, CountFold :250-318).

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
        when the sum is kept wider; bf16 to fp32 by pieces.fold_start's
        kernel)."""
        want = self.widen.get(i)
        if want is not None and t.dtype != want:
            if want == torch.float32 and t.dtype == torch.bfloat16 and t.is_cuda:
                return pieces.fold_start(t)
            return t.to(want, copy=True)
        return t.clone()

    def _add(self, i: int, t) -> None:
        """acc[i] += t in place through pieces.fold_add: fp32 sums on its
        kernel, int64 count lanes by integer add, bf16 sums (a bf16 part
        folded with no wider dtype asked for) as the fp32 add rounded to
        bf16, torch's add_ on a bf16 tensor."""
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


class TiedRowFold:
    """runtime/accumulate.py:140-247: the step gradient of a tied table split
    across stages, folded on the Head in the stock order (acc = g_0,
    acc += g_i, g_i = h_i + e_i with e_i = +0 outside the microbatch's rows)
    without a dense table per microbatch in flight.  A row takes h_i + 0.0
    as soon as no earlier microbatch still holds it; the rest of h_i waits
    for the embedding rows e_i, and the held rows resolve in microbatch order
    as h_i + e_i.  Every row sees exactly the stock sequence of adds, so the
    result is the stock fold bit for bit.

    add_head(mb, h, rows): h the (n_rows, d) gradient of the Head's use (fp32
    or bf16, on the GPU), rows T_mb (ascending unique ids, int64).
    add_embed(mb, e_rows): e_mb[T_mb] in ascending id.  Either may come
    first; out-of-order microbatches wait.  The row bookkeeping (which rows
    are held) runs on the host in numpy; one launch takes a Head gradient
    (ely_rows_split: its free rows fold, its held rows are copied out), and
    the held rows resolve in one launch of the row fold (ely_rows_fold) that
    reads the embedding rows in place, by index."""

    def __init__(self, n_rows: int, order) -> None:
        self.n_rows = int(n_rows)
        if not 0 <= self.n_rows < 2**31:
            raise ValueError(f"tied fold: a table of {self.n_rows} rows (the row slots are int32)")
        self.order = list(order)
        self.pos = 0  # next position of `order` whose Head gradient is taken
        self.acc = torch.empty(0)  # allocated by the first Head gradient
        self.first = True  # no row folded yet: microbatch order[0] assigns
        self.heads: dict = {}  # mb -> (h, rows) waiting for its prefix
        self.embeds: dict = {}  # mb -> e_rows until its held rows resolve
        # [(mb, held row ids, the same on the GPU, h on them, T_mb, first, each
        # held row's place in T_mb or -1 on the GPU)], oldest first
        self.held: list = []
        # held-row multiplicity; the row bookkeeping runs in numpy (torch's CPU
        # nonzero over a 32,768-row mask took ~0.1 ms a call)
        self.pend = np.zeros(self.n_rows, dtype=np.int32)

    def add_head(self, mb: int, h: torch.Tensor, rows: torch.Tensor) -> None:
        if mb in self.heads or self._done(mb):
            raise RuntimeError(f"tied fold: a second Head gradient for microbatch {mb}")
        if h.dim() != 2 or h.shape[0] != self.n_rows:
            raise RuntimeError(f"tied fold: Head gradient of mb {mb} has shape {tuple(h.shape)}")
        _lib.require_gpu(h, "tied fold")
        _lib.dtype_code(h)
        self.heads[mb] = (h.contiguous(), np.ascontiguousarray(rows.to(torch.int64).cpu().numpy()))
        self._advance()

    def add_embed(self, mb: int, e_rows: torch.Tensor) -> None:
        if mb in self.embeds or (self._done(mb) and not any(held[0] == mb for held in self.held)):
            raise RuntimeError(f"tied fold: a second embedding gradient for microbatch {mb}")
        self.embeds[mb] = e_rows
        self._advance()

    def _done(self, mb) -> bool:
        return mb in self.order[: self.pos]

    def _advance(self) -> None:
        while True:
            if self.held and self.held[0][0] in self.embeds:
                self._resolve()
                continue
            if self.pos < len(self.order) and self.order[self.pos] in self.heads:
                self._take_head()
                continue
            return

    def _fold_rows(self, a, a_rows_d, b, b_rows_d, idx_d, n_idx: int, first: bool, stream) -> None:
        """acc[idx] (=|+=) a[a_rows, or row j] + (b[b_rows, or row j], or
        +0.0 where b_rows is negative or there is no b), one launch; every
        index list already on the GPU."""
        if n_idx == 0:
            return
        L = _lib.load()
        _lib.check(L.ely_rows_fold(self.acc.data_ptr(), a.data_ptr(), None if a_rows_d is None else a_rows_d.data_ptr(),
                                   None if b is None else b.data_ptr(), None if b_rows_d is None else b_rows_d.data_ptr(),
                                   idx_d.data_ptr(), n_idx, self.n_rows, a.shape[0], 0 if b is None else b.shape[0],
                                   self.acc.shape[1], _lib.dtype_code(self.acc), int(first), stream),
                   "tied fold")

    def _take_head(self) -> None:
        mb = self.order[self.pos]
        h, rows = self.heads.pop(mb)
        if self.first:
            self.acc = torch.empty_like(h)
        n = self.n_rows
        if rows.size and (int(rows.min()) < 0 or int(rows.max()) >= n):
            raise RuntimeError(f"tied fold: rows of mb {mb} outside [0, {n})")
        mask = self.pend > 0
        mask[rows] = True
        keep = np.flatnonzero(mask)
        k = keep.size
        # each held row's place among the microbatch's rows, -1 for a row it
        # did not touch (that row adds +0.0 when it resolves)
        at = np.full(n, -1, dtype=np.int64)
        at[rows] = np.arange(rows.size, dtype=np.int64)
        # one upload per Head gradient: the held rows, their places and each
        # row's slot among the held ones (-1: free), packed in one pinned block
        # (from torch's pinned-memory cache, which keeps it until the copy on
        # this stream is done)
        stage = torch.empty(2 * k + (n + 1) // 2, dtype=torch.int64, pin_memory=True)
        host = stage.numpy()
        host[:k] = keep
        host[k : 2 * k] = at[keep]
        slot = host[2 * k :].view(np.int32)[:n]
        slot.fill(-1)
        slot[keep] = np.arange(k, dtype=np.int32)
        dev = h.device
        up = stage.to(dev, non_blocking=True)
        keep_d, b_rows_d, slot_d = up[:k], up[k : 2 * k], up[2 * k :].view(torch.int32)
        # free rows: acc = h + 0.0 (first) or acc + (h + 0.0); held rows:
        # copied out of h (bit for bit) so that h itself can go; one pass
        hk = torch.empty((k, h.shape[1]), dtype=h.dtype, device=dev)
        L = _lib.load()
        _lib.check(L.ely_rows_split(self.acc.data_ptr(), h.data_ptr(), slot_d.data_ptr(), hk.data_ptr() if k else None,
                                    n, k, h.shape[1], _lib.dtype_code(self.acc), int(self.first), _lib.stream_ptr(dev)),
                   "tied fold")
        self.held.append((mb, keep, keep_d, hk, rows, self.first, b_rows_d))
        self.pend[keep] += 1
        self.first = False
        self.pos += 1

    def _resolve(self) -> None:
        mb, keep, keep_d, hk, rows, first, b_rows_d = self.held.pop(0)
        e_rows = self.embeds.pop(mb)
        if e_rows.dim() != 2 or e_rows.shape[0] != rows.size or e_rows.shape[1:] != hk.shape[1:]:
            raise RuntimeError(
                f"tied fold: embedding rows of mb {mb} have shape {tuple(e_rows.shape)}, "
                f"want ({rows.size}, {tuple(hk.shape[1:])})"
            )
        e = e_rows.to(hk.device, hk.dtype).contiguous() if rows.size else None
        # held rows: acc = hk + e_on (first) or acc + (hk + e_on)
        self._fold_rows(hk, None, e, None if e is None else b_rows_d, keep_d, keep.size, first, _lib.stream_ptr(hk.device))
        self.pend[keep] -= 1

    def complete(self) -> bool:
        return self.pos == len(self.order) and not self.held

    def result(self) -> torch.Tensor:
        if not self.complete():
            raise RuntimeError(
                f"tied fold incomplete: {self.pos}/{len(self.order)} Head gradients, "
                f"{len(self.held)} microbatch(es) waiting for embedding rows"
            )
        return self.acc


class CountFold:
    """runtime/accumulate.py:250-318: the int64 selection counts of one
    step at a bias's owner, one (E,) vector per (microbatch, MoE layer),
    checked on arrival and summed by integer add in microbatch order on the
    host (exact, order-free).  The reference's refusals, named by
    (step, mb, layer, peer): a microbatch outside [0, n_mb), a layer without
    a bias here, a vector given twice, not int64, of the wrong shape, with a
    negative count or (when `total` is given) not summing to T_mb * k; and,
    at result(), a missing vector."""

    def __init__(self, step: int, n_mb: int, layers, experts: dict, total: dict | None) -> None:
        self.step = step
        self.n_mb = n_mb
        self.layers = list(layers)
        self.experts = dict(experts)  # layer -> E
        self.total = total  # layer -> T_mb * k, or None
        self.got: dict = {}  # (mb, layer) -> vector

    def _name(self, mb, layer, peer) -> str:
        return f"(step {self.step}, mb {mb}, layer {layer}, peer {peer})"

    def add(self, mb, layer, vec, peer) -> None:
        name = self._name(mb, layer, peer)
        if type(mb) is not int or not 0 <= mb < self.n_mb:
            raise RuntimeError(f"MOE-COUNT {name}: microbatch outside [0, {self.n_mb})")
        if layer not in self.experts:
            raise RuntimeError(f"MOE-COUNT {name}: no selection bias of that layer here")
        if (mb, layer) in self.got:
            raise RuntimeError(f"MOE-COUNT {name}: count vector given twice")
        if not isinstance(vec, torch.Tensor) or vec.dtype != torch.int64:
            raise RuntimeError(f"MOE-COUNT {name}: not an int64 vector")
        if tuple(vec.shape) != (self.experts[layer],):
            raise RuntimeError(f"MOE-COUNT {name}: shape {tuple(vec.shape)}, want ({self.experts[layer]},)")
        v = vec.detach().to("cpu", copy=True)
        if bool((v < 0).any()):
            raise RuntimeError(f"MOE-COUNT {name}: a negative count")
        if self.total is not None and int(v.sum()) != self.total[layer]:
            raise RuntimeError(f"MOE-COUNT {name}: counts sum to {int(v.sum())}, want T_mb*k = {self.total[layer]}")
        self.got[(mb, layer)] = v

    def missing(self) -> list:
        return [(mb, layer) for layer in self.layers for mb in range(self.n_mb) if (mb, layer) not in self.got]

    def complete(self) -> bool:
        return not self.missing()

    def result(self) -> dict:
        """{layer: int64 (E,)}: the sum over microbatches in index order."""
        gone = self.missing()
        if gone:
            mb, layer = gone[0]
            raise RuntimeError(f"MOE-COUNT {self._name(mb, layer, '-')}: count vector missing at the owner ({len(gone)} missing)")
        out = {}
        for layer in self.layers:
            acc = self.got[(0, layer)].clone()
            for mb in range(1, self.n_mb):
                acc += self.got[(mb, layer)]
            out[layer] = acc
        return out
