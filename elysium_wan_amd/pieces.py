"""The elementwise kernels and the optimizer of the sharded "pieces" update
on MI355X: the drop-in for wantrain's runtime/pieces.py:192-256 (same names
and semantics).

cast_piece: fp32 master -> working copy (bf16 RNE, or a plain copy for fp32).
fold_start / fold_add / fold: the fixed-order fp32 gradient fold, widening
bf16 parts exactly.  int64 count lanes stay on torch's exact integer add, as
the reference does (runtime/pieces.py:198-214).
adamw / step_unit: the reference's AdamW over master pieces (the fused
kernel in torch's op order) and the per-unit step.
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence

import torch

from . import _lib
from . import optim as _optim


def cast_piece(p: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """runtime/pieces.py:192-195: a new tensor, never an alias of the master."""
    if dtype == torch.bfloat16 and p.dtype == torch.float32:
        _lib.require_gpu(p, "cast_piece")
        src = p.detach().contiguous()
        out = torch.empty(src.shape, dtype=torch.bfloat16, device=src.device)
        L = _lib.load()
        _lib.check(L.ely_cast_bf16(src.data_ptr(), out.data_ptr(), src.numel(), _lib.stream_ptr(src.device)), "cast_piece")
        return out
    if dtype == p.dtype:
        return p.detach().clone()
    raise TypeError(f"cast_piece on MI355X casts float32 to bfloat16 (or copies), not {p.dtype} -> {dtype}")


def fold_start(g: torch.Tensor) -> torch.Tensor:
    """runtime/pieces.py:198-203: the fp32 accumulator, a copy of microbatch
    0's widened gradient (an int64 count lane stays int64)."""
    if g.dtype == torch.int64:
        return g.clone()
    _lib.require_gpu(g, "fold_start")
    if g.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"fold_start widens float32 or bfloat16 gradients, got {g.dtype}")
    if g.dtype == torch.float32:
        return g.detach().clone()
    # widening is exact: the fp32 value of a bf16 is its bits moved to the top
    src = g.detach().contiguous()
    out = torch.empty(src.shape, dtype=torch.float32, device=src.device)
    L = _lib.load()
    _lib.check(L.ely_widen_bf16(src.data_ptr(), out.data_ptr(), src.numel(), _lib.stream_ptr(src.device)), "fold_start")
    return out


def fold_add(acc: torch.Tensor, g: torch.Tensor) -> None:
    """runtime/pieces.py:206-214: acc += widen(g), one fp32 rounding per
    element.  An accumulator that is not fold_start's fp32 (a bf16 one) takes
    the reference's in-place add as torch computes it there: the fp32 sum
    rounded to bf16 (ely_fold_add_bf16)."""
    if acc.dtype == torch.int64:
        if g.dtype != torch.int64:
            raise ValueError(f"a count lane folds int64 only, got {g.dtype}")
        acc.add_(g)
        return
    _lib.require_gpu(acc, "fold_add")
    if acc.dtype not in (torch.float32, torch.bfloat16) or not acc.is_contiguous():
        raise ValueError("fold_add accumulates into a contiguous float32 (or bfloat16) tensor")
    g = g.detach().contiguous()
    if g.numel() != acc.numel() or g.device != acc.device:
        raise ValueError("fold_add: gradient and accumulator differ in size or device")
    L = _lib.load()
    fn = L.ely_fold_add if acc.dtype == torch.float32 else L.ely_fold_add_bf16
    _lib.check(fn(acc.data_ptr(), g.data_ptr(), _lib.dtype_code(g), acc.numel(), _lib.stream_ptr(acc.device)), "fold_add")


def fold(gs: Iterable[torch.Tensor]) -> torch.Tensor:
    """runtime/pieces.py:217-227: left fold in microbatch-index order."""
    acc = None
    for g in gs:
        if acc is None:
            acc = fold_start(g)
        else:
            fold_add(acc, g)
    if acc is None:
        raise ValueError("a fold over zero microbatches")
    return acc


def adamw(params: Iterable[torch.Tensor], lr: float):
    """runtime/pieces.py:230-232: the reference's optimizer over owned pieces
    -- torch.optim.AdamW(lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0),
    here the fused kernel in torch's op order."""
    return _optim.build("adamw", params, lr)


def step_unit(opt, params: Sequence[torch.Tensor], grads: Sequence[torch.Tensor]) -> None:
    """runtime/pieces.py:235-256: one unit's update.  Only `params` carry
    gradients during the step, so every other parameter's state and step
    counter are left untouched; gradients are cleared afterwards."""
    if len(params) != len(grads):
        raise ValueError(f"{len(params)} params, {len(grads)} grads")
    ids = {id(p) for p in params}
    held = {id(p) for group in opt.param_groups for p in group["params"]}
    if not ids <= held:
        raise ValueError("step_unit: a parameter outside this optimizer")
    for group in opt.param_groups:
        for p in group["params"]:
            if id(p) not in ids:
                p.grad = None
    if isinstance(opt, _optim.FusedAdamW):
        # bf16 gradients cannot sit in an fp32 parameter's .grad: hand them in
        by_id = {id(p): g for p, g in zip(params, grads)}
        opt.step(grads=[by_id.get(id(p)) for p in opt.params])
    else:
        for p, g in zip(params, grads):
            p.grad = g
        opt.step()
    for p in params:
        p.grad = None
