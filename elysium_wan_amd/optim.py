"""The stage optimizer on MI355X: the drop-in for wantrain's runtime/optim.py.

`build(optimizer, params, lr)` keeps the reference's names and recipes
(runtime/optim.py:32-69):

* "adamw"      -> FusedAdamW(order="torch"): torch.optim.AdamW's arithmetic
                  (TORCH/optim/adam.py:554-800), within 1 ulp of it
                  (bit for bit torch's GPU foreach kernels on this image).
* "adamw-host" -> FusedAdamW(order="host", moments="host"): HostAdamW's
                  single-rounding op order (runtime/optim.py:277-298), bit for
                  bit, with its moments in pinned host memory streamed through
                  the GPU in chunks (runtime/optim.py:176-204, 301-363).
                  moments="device" keeps them in HBM instead: a 288 GB
                  MI355X holds a stage's fp32 p/m/v/g, and the step is then
                  HBM-bound rather than PCIe-bound.

Either way one step is at most two launches over the whole parameter list:
the deterministic grad-norm (when max_norm is set) and the fused
clip + AdamW + bf16-working-copy kernel, one HBM pass per element.  With
step(on_param=...) the update goes out in parameter-ordered groups instead,
each followed by on_param of its parameters, so a caller can release layers
as they land.

The torch.optim surface the runtime uses is kept: step(on_param=None),
zero_grad, state_dict, load_state_dict (torch's AdamW layout: state[i] =
{step, exp_avg, exp_avg_sq}, one param group; "moments": "host" for
adamw-host), param_groups and state (keyed by parameter index for
adamw-host, as HostAdamW, and by parameter tensor for adamw, as torch).
"""

from __future__ import annotations

import math
import weakref
from collections.abc import Iterable, MutableMapping

import numpy as np
import torch

from . import _lib

OPTIMIZERS = ("adamw", "adamw-host")
CHUNK = 1 << 24  # the reference's streamed chunk (runtime/optim.py:33); kept for callers that read it
STATE_BYTES = {"adamw": 16, "adamw-host": 8}
# runtime/spec.py:27: the AdamW every stage and the reference run.
ADAMW = {"betas": (0.9, 0.95), "eps": 1e-8, "weight_decay": 0.0}
_ALIGN = 64  # moment views start on 256-byte boundaries of the flat buffers


def state_bytes_per_param(optimizer: str = "adamw") -> int:
    """runtime/optim.py:39-42: device bytes per trainable element the
    reference's planner charges for each recipe."""
    if optimizer not in STATE_BYTES:
        raise ValueError(f"optimizer {optimizer!r} is not one of {OPTIMIZERS}")
    return STATE_BYTES[optimizer]


def build(optimizer: str, params: Iterable[torch.Tensor], lr: float, **kw):
    """runtime/optim.py:45-54: the optimizer a stage and the reference
    construct over their trainable parameters, in order."""
    if optimizer == "adamw":
        return FusedAdamW(params, lr=lr, order="torch", **{**ADAMW, **kw})
    if optimizer == "adamw-host":
        # the reference's memory contract (8 device bytes per element): moments
        # in host memory, streamed through the GPU; moments="device" keeps them in HBM
        return HostAdamW(params, lr=lr, **{**ADAMW, **kw})
    raise ValueError(f"optimizer {optimizer!r} is not one of {OPTIMIZERS}")


def _torch_adamw_group() -> dict:
    """The param group torch's AdamW records for the reference's constants,
    without its "params" and "lr".  Read once, when this module loads: a
    torch optimizer's constructor leaves collectable reference cycles among
    its frames, and one built inside FusedAdamW.__init__ would tie the new
    optimizer (its parameters and moments) to them until the garbage
    collector runs."""
    probe = torch.optim.AdamW([torch.zeros(1, requires_grad=True)], lr=1e-3, **ADAMW)
    return {k: v for k, v in probe.state_dict()["param_groups"][0].items() if k not in ("params", "lr")}


_TORCH_ADAMW_GROUP = _torch_adamw_group()


def hparams(lr: float, optimizer: str = "adamw") -> dict:
    """runtime/optim.py:57-69: the param-group hyperparameters a checkpoint
    records, read off torch's own AdamW defaults (keys in torch's order)."""
    group = {"lr": lr, **_TORCH_ADAMW_GROUP}
    if optimizer == "adamw-host":
        group["moments"] = "host"
    elif optimizer != "adamw":
        raise ValueError(f"optimizer {optimizer!r} is not one of {OPTIMIZERS}")
    return group


def json_norm(group: dict) -> dict:
    """runtime/optim.py:366-369: tuples as lists, so a group read back from
    JSON or torch.load compares equal to a fresh one."""
    return {k: (list(v) if isinstance(v, tuple) else v) for k, v in sorted(group.items())}


def _f32(x: float) -> float:
    """A double rounded once to fp32 (runtime/optim.py:72-74)."""
    return float(np.float32(x))


def host_consts(lr: float, betas, eps: float, weight_decay: float, t: float) -> list:
    """HostAdamW.step's per-step constants (runtime/optim.py:158-167), each
    computed in double and rounded once to fp32."""
    b1, b2 = betas
    return [
        _f32(1.0 - lr * weight_decay),
        _f32(b1),
        _f32(1.0 - b1),
        _f32(b2),
        _f32(1.0 - b2),
        _f32(1.0 / math.sqrt(1.0 - b2**t)),
        _f32(eps),
        _f32(lr / (1.0 - b1**t)),
    ]


def torch_consts(lr: float, betas, eps: float, weight_decay: float, t: float) -> list:
    """The fp32 scalars torch's _multi_tensor_adam hands its kernels for step
    t (TORCH/optim/adam.py:689-800): decay, 1-b1, b2, 1-b2, bc2**0.5, eps,
    (lr/bc1)*-1."""
    b1, b2 = betas
    bc1 = 1 - b1**t
    bc2 = 1 - b2**t
    return [
        _f32(1 - lr * weight_decay),
        _f32(1 - b1),
        _f32(b2),
        _f32(1 - b2),
        _f32(bc2**0.5),
        _f32(eps),
        _f32((lr / bc1) * -1),
        0.0,
    ]


class _State(MutableMapping):
    """`opt.state`, keyed as each recipe's reference keys it:
    parameter indices for "adamw-host" (HostAdamW, runtime/optim.py:106) and
    the parameter tensors themselves for "adamw" (torch.optim.AdamW, whose
    state runtime/stage.py:2265-2271 reads and :2642-2646 assigns per master
    tensor).  Either kind of key is accepted for lookup.  An entry is
    {step, exp_avg, exp_avg_sq}; the moments are views of the optimizer's own
    storage, so assigning an entry copies the given values into it (the
    optimizer never adopts the caller's tensors), and deleting one makes the
    parameter start again from zero moments at step 0."""

    def __init__(self, opt: FusedAdamW):
        # a weak reference: the optimizer owns this mapping, and a cycle
        # would keep its parameters and moments alive after `del opt` until
        # the garbage collector happened to run
        self._ref = weakref.ref(opt)

    @property
    def _opt(self) -> FusedAdamW:
        opt = self._ref()
        if opt is None:
            raise ReferenceError("the optimizer of this state no longer exists")
        return opt

    def _index(self, key) -> int:
        opt = self._opt
        if isinstance(key, torch.Tensor):
            i = opt._pindex.get(id(key))
            if i is None or opt.params[i] is not key:
                raise KeyError("a tensor that is not a parameter of this optimizer")
            return i
        if isinstance(key, (int, np.integer)) and not isinstance(key, bool) and 0 <= int(key) < len(opt.params):
            return int(key)
        raise KeyError(key)

    def __getitem__(self, key) -> dict:
        return self._opt._st[self._index(key)]

    def __setitem__(self, key, value) -> None:
        i = self._index(key)
        self._opt._assign(i, value)

    def __delitem__(self, key) -> None:
        i = self._index(key)
        del self._opt._st[i]

    def __contains__(self, key) -> bool:
        try:
            return self._index(key) in self._opt._st
        except KeyError:
            return False

    def __iter__(self):
        opt = self._opt
        for i in sorted(opt._st):
            yield opt.params[i] if opt.order == "torch" else i

    def __len__(self) -> int:
        return len(self._opt._st)

    def __repr__(self) -> str:
        return f"{type(self).__name__}({len(self)} entries, keyed by {'parameter' if self._opt.order == 'torch' else 'index'})"


class FusedAdamW:
    """AdamW (decoupled weight decay, no amsgrad) over a ragged list of fp32
    CUDA parameters, one fused launch per step.

    order: "host" (HostAdamW's bits) or "torch" (torch.optim.AdamW's op order).
    max_norm: clip the global L2 norm of the gradients to this value before
        the update (torch.nn.utils.clip_grad_norm_'s coefficient), fused into
        the same launch; None disables clipping.
    working_copy: None, True (allocate a bf16 copy of every trainable
        parameter) or a list of bf16 tensors shaped like the parameters;
        refreshed with the RNE bf16 cast of the updated parameter
        (pieces.cast_piece) in the update's own pass.
    moments: "device" (HBM) or "host" (pinned host memory: HostAdamW's
        memory contract).  Host moments are updated in place: the fused
        kernel reads and writes them through the GPU's mapping of the pinned
        buffers, PCIe busy in both directions at once.  pipeline=True
        instead streams them through the GPU in `chunk`-element pieces over
        `slots` staging buffers (the reference's scheme), pipeline=False
        with serial copies; the bits are the same either way.
    Gradients (p.grad, or step(grads=...)) may be float32 or bfloat16 (the
    bf16 fold start of runtime/pieces.py:198-203 happens in registers);
    step(acc=...) folds the last microbatch into fp32 accumulators inside the
    update.  Moments exist for trainable (requires_grad) parameters only,
    allocated at the first step, as the reference allocates them per stepped
    parameter.
    release_elems: with step(on_param=...), the update is issued in
        parameter-ordered groups of at least this many elements, and
        on_param(i) runs as soon as the group holding parameter i is issued,
        so a caller can release each layer while later ones still update
        (runtime/optim.py:164-170, runtime/stage.py:3080-3099).  Without
        on_param the step is one launch per gradient dtype.  The bits are the
        same either way.
    """

    def __init__(
        self,
        params: Iterable[torch.Tensor],
        lr: float,
        betas: tuple = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 0.0,
        *,
        order: str = "host",
        max_norm: float | None = None,
        working_copy=None,
        moments: str = "device",
        chunk: int = CHUNK,
        pipeline: bool | None = None,
        slots: int = 3,
        release_elems: int = 1 << 26,
    ):
        self.params = list(params)
        self._pindex = {id(p): i for i, p in enumerate(self.params)}
        self.release_elems = max(1, int(release_elems))
        if order not in ("host", "torch"):
            raise ValueError(f"order {order!r} is not 'host' or 'torch'")
        if moments not in ("device", "host"):
            raise ValueError(f"moments {moments!r} is not 'device' or 'host'")
        if int(chunk) < 1 or int(slots) < 1:
            raise ValueError("chunk and slots are positive")
        self.moments = moments
        self.chunk, self.pipeline, self.slots = int(chunk), pipeline, int(slots)
        self.resident: set = set()  # host mode: indices whose moments were promoted to the GPU
        self._staging = None  # host mode: per-step streaming buffers, streams and events
        # host mode, staged copies: a list to receive ("h2d" | "d2h", start,
        # end) timing-event pairs around every chunk copy, on the copy's own
        # stream (for measurement; None records nothing)
        self.copy_timing = None
        self._mapped = None  # host mode: the GPU's addresses of the pinned moment buffers
        self.order = order
        self.recipe = "adamw-host" if order == "host" else "adamw"
        if order == "torch":
            # the "adamw" recipe is torch.optim.AdamW (runtime/optim.py:50-51):
            # its argument checks and messages, hyperparameters first
            # (TORCH/optim/adamw.py -> adam.py:58-67), then the empty list
            # (TORCH/optim/optimizer.py); HostAdamW checks neither
            if not 0.0 <= lr:
                raise ValueError(f"Invalid learning rate: {lr}")
            if not 0.0 <= eps:
                raise ValueError(f"Invalid epsilon value: {eps}")
            if not 0.0 <= betas[0] < 1.0:
                raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
            if not 0.0 <= betas[1] < 1.0:
                raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
            if not 0.0 <= weight_decay:
                raise ValueError(f"Invalid weight_decay value: {weight_decay}")
            if not self.params:
                raise ValueError("optimizer got an empty parameter list")
        devices = set()
        for p in self.params:
            # a frozen tensor never has a gradient and is never stepped (runtime/optim.py:98-99)
            if p.requires_grad and p.dtype != torch.float32:
                raise ValueError(f"{self.recipe} trains fp32 parameters, got {p.dtype}")
            if p.requires_grad:
                _lib.require_gpu(p, self.recipe)
                devices.add(p.device)
        if len(devices) > 1:
            raise ValueError(f"{self.recipe}: parameters span devices {sorted(map(str, devices))}; build one optimizer per device")
        if not devices:
            # no parameter requires grad: the moments follow the GPU tensors
            devices = {p.device for p in self.params if p.device.type == "cuda"}
            if len(devices) > 1:
                raise ValueError(f"{self.recipe}: parameters span devices {sorted(map(str, devices))}; build one optimizer per device")
        # the device of the moments (set by the first stepped parameter if still unknown)
        self.device = devices.pop() if devices else None
        self.lr, self.betas, self.eps, self.weight_decay = lr, tuple(betas), eps, weight_decay
        self.max_norm = None if max_norm is None else float(max_norm)
        group = hparams(lr, self.recipe)
        group.update(lr=lr, betas=self.betas, eps=eps, weight_decay=weight_decay)
        self._group = group
        self.param_groups = [{**group, "params": self.params}]
        self._st: dict = {}  # parameter index -> {"step", "exp_avg", "exp_avg_sq"}
        self.state = _State(self)
        self._flat_m = self._flat_v = None
        self._fresh: set = set()  # indices whose flat moment slices still hold the allocation's zeros
        self._steps = None  # flat fp32 step counters; state[i]["step"] are 0-d views of it
        self._tables: dict = {}  # descriptor arrays kept between steps, per launch group (_launch_cached)
        self._norm = None  # device ely_norm_result of the last clipped step
        self.working_copies = self._init_copies(working_copy)

    # ------------------------------------------------------------ storage

    def _init_copies(self, working_copy):
        if working_copy is None:
            return None
        if working_copy is True:
            return [torch.empty(p.shape, dtype=torch.bfloat16, device=p.device) if p.requires_grad else None for p in self.params]
        copies = list(working_copy)
        if len(copies) != len(self.params):
            raise ValueError(f"{len(copies)} working copies for {len(self.params)} parameters")
        for c, p in zip(copies, self.params):
            if c is None:
                continue
            if c.dtype != torch.bfloat16 or tuple(c.shape) != tuple(p.shape) or not c.is_contiguous() or c.device != p.device:
                raise ValueError("a working copy is a contiguous bf16 tensor shaped like its parameter, on its device")
        return copies

    def _alloc_state(self) -> None:
        """Moments live in two flat fp32 buffers in parameter order, each
        tensor's slice starting on a 256-byte boundary; state[i] holds views.
        moments="device": in HBM.  moments="host": in pinned host memory
        (runtime/optim.py:121-130), streamed through the GPU at every step."""
        offs, total = [], 0
        for p in self.params:
            # frozen tensors (a LoRA base) get no slice: they are never stepped
            # through p.grad, and one stepped anyway gets its own moments (_slot)
            if not p.requires_grad:
                offs.append(None)
                continue
            offs.append(total)
            total += -(-p.numel() // _ALIGN) * _ALIGN
        dev = self.device
        if dev is None or dev.type != "cuda":
            raise ValueError(f"{self.recipe}: the moments live on the parameters' GPU, got device {dev}")
        if self.moments == "host":
            self._flat_m = torch.zeros(max(total, 1), dtype=torch.float32, pin_memory=True)
            self._flat_v = torch.zeros(max(total, 1), dtype=torch.float32, pin_memory=True)
            # the GPU's own addresses of the pinned buffers: the update then
            # reads and writes the moments in place over PCIe (both directions
            # at once) instead of copying chunks through staging buffers;
            # pipeline=True or False asks for the staged or the serial copies
            self._mapped = None
            if self.pipeline is None:
                with torch.cuda.device(dev):
                    dm, dvv = _lib.host_device_pointer(self._flat_m), _lib.host_device_pointer(self._flat_v)
                if dm is not None and dvv is not None:
                    self._mapped = (dm, dvv)
        else:
            self._flat_m = torch.zeros(max(total, 1), dtype=torch.float32, device=dev)
            self._flat_v = torch.zeros(max(total, 1), dtype=torch.float32, device=dev)
        self._offs = offs
        self._steps = torch.zeros(max(len(self.params), 1), dtype=torch.float32)
        self._fresh = {i for i, o in enumerate(offs) if o is not None}
        self._tables = {}

    def _slot(self, i: int, p: torch.Tensor, clear: bool = True) -> dict:
        """State entry i, made on first use: zero moments at step 0.  A slice
        of the flat buffers that an earlier entry used (one that
        load_state_dict or `del state[p]` dropped) is zeroed again, unless the
        caller is about to overwrite it (clear=False)."""
        st = self._st.get(i)
        if st is None:
            if self._flat_m is None:
                self._alloc_state()
            o, n = self._offs[i], p.numel()
            if o is None:
                # a tensor outside the flat layout (no requires_grad) stepped
                # through grads=: moments of its own, in HBM (taking the
                # direct path in host mode)
                m = torch.zeros(p.shape, dtype=torch.float32, device=self.device)
                v = torch.zeros(p.shape, dtype=torch.float32, device=self.device)
                if self.moments == "host":
                    self.resident.add(i)
            else:
                m = self._flat_m[o : o + n].view(p.shape)
                v = self._flat_v[o : o + n].view(p.shape)
                if clear and i not in self._fresh:
                    m.zero_()
                    v.zero_()
                self._fresh.discard(i)
            self._steps[i] = 0.0
            st = self._st[i] = {
                "step": self._steps[i],  # a 0-d view of the flat counters
                "exp_avg": m,
                "exp_avg_sq": v,
            }
        return st

    def _assign(self, i: int, st: dict) -> None:
        """Entry i set to the given {step, exp_avg, exp_avg_sq}: the values are
        copied into the optimizer's storage (a resume, runtime/stage.py:
        2642-2646, and load_state_dict)."""
        p = self.params[i]
        for k in ("exp_avg", "exp_avg_sq"):
            if tuple(st[k].shape) != tuple(p.shape):
                raise ValueError(f"optimizer state {i}.{k} has shape {tuple(st[k].shape)}")
        self._st.pop(i, None)
        slot = self._slot(i, p, clear=False)
        slot["step"].copy_(torch.as_tensor(st["step"], dtype=torch.float32).detach().cpu())
        slot["exp_avg"].copy_(st["exp_avg"])
        slot["exp_avg_sq"].copy_(st["exp_avg_sq"])

    # --------------------------------------------------------------- step

    def _consts(self, t: float, lr: float, betas, eps: float, weight_decay: float) -> list:
        if self.order == "host":
            return host_consts(lr, betas, eps, weight_decay, t)
        return torch_consts(lr, betas, eps, weight_decay, t)

    @torch.no_grad()
    def step(self, on_param=None, grads=None, acc=None) -> None:
        """One AdamW step over every parameter with a gradient, in order;
        `on_param(i)` runs right after parameter i's update is issued
        (runtime/optim.py:145-170): the update then goes out in
        parameter-ordered groups of `release_elems` elements, so a layer can
        be released while later ones still update.  Nothing here waits for
        the GPU, except that host moments land before the step returns, as
        HostAdamW's do (runtime/optim.py:171-174).

        grads: optional list aligned with the parameters (None entries skip
        a parameter) used instead of p.grad -- the way to hand in bf16
        gradients, which torch does not let an fp32 parameter's .grad hold.
        acc: optional list aligned with the parameters of fp32 fold
        accumulators (runtime/accumulate.py:93-104) holding the sum of the
        earlier microbatches; the step's gradient is then acc[i] + grads[i]
        rounded once to fp32 (pieces.fold_add), folded inside the update
        without writing acc."""
        if grads is not None and len(grads) != len(self.params):
            raise ValueError(f"{len(grads)} gradients for {len(self.params)} parameters")
        if acc is not None and len(acc) != len(self.params):
            raise ValueError(f"{len(acc)} accumulators for {len(self.params)} parameters")
        gl = [p.grad for p in self.params] if grads is None else grads
        # as torch: a parameter without a gradient is not stepped
        idx = [i for i, g in enumerate(gl) if g is not None]
        ps = [self.params[i] for i in idx]
        gs = [gl[i] for i in idx]
        accs = None if acc is None else [acc[i] for i in idx]
        self._check_inputs(idx, ps, gs, accs)
        if not idx:
            return
        sts = [self._slot(i, p) for i, p in zip(idx, ps)]
        ms = [st["exp_avg"] for st in sts]
        vs = [st["exp_avg_sq"] for st in sts]
        host = [j for j, m in enumerate(ms) if not m.is_cuda]
        if host:
            self._check_host_moments([idx[j] for j in host], [ms[j] for j in host], [vs[j] for j in host])
        # the step counters are views of one flat tensor: one increment for all
        if len(idx) == len(self.params):
            self._steps[: len(idx)] += 1
            ts = self._steps[: len(idx)].tolist()
        else:
            it = torch.tensor(idx, dtype=torch.int64)
            self._steps[it] += 1
            ts = self._steps[it].tolist()
        cs = [self.working_copies[i] for i in idx] if self.working_copies is not None else [None] * len(idx)
        lr, betas, eps, wd = self._hyper()
        per_t = {t: self._consts(t, lr, betas, eps, wd) for t in set(ts)}
        consts = [per_t[t] for t in ts]  # tensors at one step share one list object
        dev = ps[0].device
        groups = [list(range(len(idx)))] if on_param is None else self._release_groups(ps)
        # the gradients' table, built once for the norm and a launch over all of them
        garr = _lib.tensor_array(gs)
        with torch.cuda.device(dev):
            # the norm covers every gradient of the step, before any group updates
            coef_ptr = self._clip_coef(gs, accs, garr) if self.max_norm is not None else None
            for grp in groups:
                self._issue(grp, idx, ps, gs, ms, vs, cs, consts, coef_ptr, accs, wd != 0, garr)
                if on_param is not None:
                    for j in grp:
                        on_param(idx[j])
            if host:
                # the host moments are the state: they land before the step returns (runtime/optim.py:171-174)
                torch.cuda.synchronize(dev)

    def _hyper(self) -> tuple:
        """(lr, betas, eps, weight_decay) of this step: torch.optim.AdamW reads
        them from its param group at every step (so a scheduler's lr takes
        effect); HostAdamW keeps its constructor's (runtime/optim.py:100)."""
        if self.order == "torch":
            g = self.param_groups[0]
            b1, b2 = g["betas"]
            return float(g["lr"]), (float(b1), float(b2)), float(g["eps"]), float(g["weight_decay"])
        return self.lr, self.betas, self.eps, self.weight_decay

    def _release_groups(self, ps) -> list:
        """Consecutive runs of stepped parameters, each closed once it holds
        release_elems elements (the last may hold fewer)."""
        groups, cur, n = [], [], 0
        for j, p in enumerate(ps):
            cur.append(j)
            n += p.numel()
            if n >= self.release_elems:
                groups.append(cur)
                cur, n = [], 0
        if cur:
            groups.append(cur)
        return groups

    def _issue(self, grp, idx, ps, gs, ms, vs, cs, consts, coef_ptr, accs, wd: bool, garr=None) -> None:
        """The update of the stepped parameters at positions `grp`: one launch
        per gradient dtype for HBM moments (torch groups by dtype the same
        way), then the host moments' update (in place through the mapping,
        or staged).  garr: the table of all the step's gradients, reused by
        a launch that covers them all."""
        direct = [j for j in grp if ms[j].is_cuda]
        streamed = [j for j in grp if not ms[j].is_cuda]
        for gdt in (torch.bfloat16, torch.float32):
            sel = [j for j in direct if gs[j].dtype == gdt]
            if sel:
                whole = garr if len(sel) == len(gs) else None
                self._launch_cached(sel, idx, ps, gs, ms, vs, cs, consts, coef_ptr, accs, wd, whole)
        if streamed:
            sub = lambda xs: [xs[j] for j in streamed]  # noqa: E731
            if self._mapped is not None:
                self._update_mapped(sub(ps), sub(gs), sub(ms), sub(vs), sub(cs), sub(consts), coef_ptr,
                                    None if accs is None else sub(accs), wd)
            else:
                self._stream_host_moments(sub(idx), sub(ps), sub(gs), sub(cs), sub(consts), coef_ptr,
                                          None if accs is None else sub(accs), wd)

    _GRAD_DTYPES = (torch.float32, torch.bfloat16)

    def _check_inputs(self, idx, ps, gs, accs) -> None:
        """The reference's refusals (runtime/optim.py:98-99, 177-178) plus the
        GPU-side contract, one pass over the stepped parameters."""
        f32, gdts = torch.float32, self._GRAD_DTYPES
        # devices compared by index (get_device(): -1 off the GPU), the
        # cheapest of torch's device queries in this per-tensor loop
        want = -2 if self.device is None else (self.device.index if self.device.type == "cuda" else -1)
        for k, (i, p, g) in enumerate(zip(idx, ps, gs)):
            if p.dtype != f32:
                raise ValueError(f"{self.recipe} trains fp32 parameters, got {p.dtype}")
            if not p.is_contiguous():
                raise ValueError(f"{self.recipe} steps contiguous parameters only")
            pdi = p.get_device()
            if g.get_device() != pdi or g.shape != p.shape or not g.is_contiguous():
                raise ValueError(f"{self.recipe}: the gradient of parameter {i} must be contiguous, shaped like it, on its device")
            if g.dtype not in gdts:
                raise ValueError(f"{self.recipe}: gradients are float32 or bfloat16, got {g.dtype}")
            if pdi < 0:
                _lib.require_gpu(p, self.recipe)
            if want == -2:
                self.device, want = p.device, pdi
            elif pdi != want:
                raise ValueError(f"{self.recipe}: parameter {i} is on {p.device}, the optimizer's moments on {self.device}")
            if accs is not None:
                a = accs[k]
                if a is None or a.dtype != f32 or a.shape != p.shape or not a.is_contiguous() or a.get_device() != pdi:
                    raise ValueError(f"{self.recipe}: the fold accumulator of parameter {i} must be a contiguous float32 tensor shaped like it, on its device")

    def _launch_cached(self, sel, idx, ps, gs, ms, vs, cs, consts, coef_ptr, accs, wd: bool, garr=None) -> None:
        """_launch over the stepped parameters at positions `sel`, with the
        descriptor arrays of the parameters, moments and working copies kept
        from the last launch of the same parameters while every one of their
        data pointers is unchanged (a state entry replaced, a promote or a
        load_state_dict moves the moments, and the arrays are rebuilt).
        Gradients and accumulators are new every step."""
        key = tuple(idx[j] for j in sel)
        ptrs = [ps[j].data_ptr() for j in sel]
        ptrs += [ms[j].data_ptr() for j in sel]
        ptrs += [vs[j].data_ptr() for j in sel]
        ptrs += [0 if cs[j] is None else cs[j].data_ptr() for j in sel]
        t = self._tables.get(key)
        if t is None or t["ptrs"] != ptrs:
            if len(self._tables) >= 64:
                self._tables.clear()
            copies = [(_lib.ely_tensor(cs[j]) if cs[j] is not None else _lib.ElyTensor(None, 0, _lib.BF16, 0)) for j in sel]
            t = self._tables[key] = {
                "ptrs": ptrs,
                "p": _lib.tensor_array([ps[j] for j in sel]),
                "m": _lib.tensor_array([ms[j] for j in sel]),
                "v": _lib.tensor_array([vs[j] for j in sel]),
                "c": _lib.tensor_array(copies),
            }
        self._launch_arrays(len(sel), t["p"], garr if garr is not None else _lib.tensor_array([gs[j] for j in sel]),
                            t["m"], t["v"], t["c"], [consts[j] for j in sel], coef_ptr,
                            None if accs is None else _lib.tensor_array([accs[j] for j in sel]), ps[sel[0]].device, wd)

    def _check_host_moments(self, idx, ms, vs) -> None:
        """Host moments are views of the optimizer's two pinned buffers (the
        update reads and writes them there, in place or through the staging
        copies); a state tensor swapped for another host tensor is refused
        before any launch."""
        for name, flat, ts in (("exp_avg", self._flat_m, ms), ("exp_avg_sq", self._flat_v, vs)):
            lo, hi = flat.data_ptr(), flat.data_ptr() + flat.numel() * 4
            for i, t in zip(idx, ts):
                a = t.data_ptr()
                if not (t.dtype == torch.float32 and t.is_contiguous() and lo <= a and a + t.numel() * 4 <= hi):
                    raise ValueError(f"{self.recipe}: state[{i}][{name!r}] is not a view of the optimizer's pinned moment buffer")

    def _update_mapped(self, ps, gs, ms, vs, cs, consts, coef_ptr, accs, wd: bool) -> None:
        """The update of parameters whose moments live in pinned host memory,
        in place: the fused kernel gets the moments' addresses as the GPU
        sees the mapped buffers, and its loads and stores of m and v cross
        PCIe in both directions at once (one launch per gradient dtype)."""
        (dm, dv), hm, hv = self._mapped, self._flat_m.data_ptr(), self._flat_v.data_ptr()
        mapped = lambda t, dbase, hbase: _lib.ElyTensor(dbase + (t.data_ptr() - hbase), t.numel(), _lib.F32, 0)  # noqa: E731
        for gdt in (torch.bfloat16, torch.float32):
            sel = [j for j in range(len(ps)) if gs[j].dtype == gdt]
            if not sel:
                continue
            self._launch([ps[j] for j in sel], [gs[j] for j in sel], [mapped(ms[j], dm, hm) for j in sel],
                         [mapped(vs[j], dv, hv) for j in sel], [cs[j] for j in sel], [consts[j] for j in sel], coef_ptr,
                         None if accs is None else [accs[j] for j in sel], wd)

    def _stream_host_moments(self, idx, ps, gs, cs, consts, coef_ptr, accs, wd: bool) -> None:
        """The update of parameters whose moments live in host memory
        (runtime/optim.py:176-204, 301-363): the flat moment buffers are cut
        into equal chunks of `chunk` elements along parameter order (a chunk
        spans as many parameters as it overlaps); chunk k goes through
        staging slot k % slots.  Its copy in, its update (with the launch's small
        table upload) and the release of the slot run in order on the upload
        stream; its copy out runs on the download stream once the update is
        done, so the next chunk's copy in and this one's copy out overlap
        (PCIe is full duplex).  Keeping each chunk's table upload behind its
        own copy in, on one stream, measured faster than updating on the
        caller's stream, where the small uploads waited behind the bulk
        copies.  With pipeline=False everything runs on the current stream."""
        dev = self.device
        chunk = self.chunk
        # runs of stepped parameters adjacent in the flat buffers (only the
        # 256-byte alignment between them), each cut into equal chunks of the
        # flat buffer: a chunk updates every parameter piece it overlaps, so
        # the pipeline moves full chunks instead of one per tensor boundary
        runs = []  # [flat start, flat end, stepped parameters]
        for o, j in sorted((self._offs[idx[j]], j) for j in range(len(ps))):
            n = ps[j].numel()
            if runs and o - runs[-1][1] < _ALIGN:
                runs[-1][1] = o + n
                runs[-1][2].append(j)
            else:
                runs.append([o, o + n, [j]])
        groups = []  # [flat start, flat end, pieces (j, s, e): elements [s, e) of stepped parameter j]
        for a0, b0, js in runs:
            for a in range(a0, b0, chunk):
                b = min(a + chunk, b0)
                members = []
                for j in js:
                    o = self._offs[idx[j]]
                    s0, e0 = max(a, o) - o, min(b, o + ps[j].numel()) - o
                    if s0 < e0:
                        members.append((j, s0, e0))
                groups.append([a, b, members])
        staged = self.pipeline is not False
        st = self._staging_buffers(dev, max(b - a for a, b, _ in groups))
        caller = torch.cuda.current_stream(dev)
        up, down = (st["h2d"], st["d2h"]) if staged else (caller, caller)
        if staged:
            # the gradients, the clip coefficient and earlier updates are the caller's
            up.wait_stream(caller)
        mh, vh = self._flat_m, self._flat_v
        for k, (a, b, members) in enumerate(groups):
            slot = k % len(st["bufs"])
            md, vd = st["bufs"][slot][0][: b - a], st["bufs"][slot][1][: b - a]
            if staged and st["used"][slot]:
                up.wait_event(st["ev_back"][slot])
            with torch.cuda.stream(up):
                self._timed_copy(md, mh[a:b], "h2d", up)
                self._timed_copy(vd, vh[a:b], "h2d", up)
                for gdt in (torch.bfloat16, torch.float32):
                    sel = [(j, s0, e0) for j, s0, e0 in members if gs[j].dtype == gdt]
                    if not sel:
                        continue
                    views = lambda ts: [ts[j].view(-1)[s0:e0] for j, s0, e0 in sel]  # noqa: E731
                    off = [self._offs[idx[j]] - a for j, _, _ in sel]
                    self._launch(
                        views(ps), views(gs),
                        [md[o + s0 : o + e0] for o, (_, s0, e0) in zip(off, sel)],
                        [vd[o + s0 : o + e0] for o, (_, s0, e0) in zip(off, sel)],
                        [None if cs[j] is None else cs[j].view(-1)[s0:e0] for j, s0, e0 in sel],
                        [consts[j] for j, _, _ in sel], coef_ptr,
                        None if accs is None else views(accs), wd,
                    )
                if staged:
                    st["ev_done"][slot].record(up)
            if staged:
                down.wait_event(st["ev_done"][slot])
            with torch.cuda.stream(down):
                self._timed_copy(mh[a:b], md, "d2h", down)
                self._timed_copy(vh[a:b], vd, "d2h", down)
                if staged:
                    st["ev_back"][slot].record(down)
            st["used"][slot] = staged
        if staged:
            caller.wait_stream(up)
            caller.wait_stream(down)
            st["used"] = [False] * len(st["bufs"])

    def _timed_copy(self, dst, src, what: str, stream) -> None:
        """dst.copy_(src) on the current stream, between timing events when
        copy_timing is a list."""
        tm = self.copy_timing
        if tm is None:
            dst.copy_(src, non_blocking=True)
            return
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        dst.copy_(src, non_blocking=True)
        e1.record(stream)
        tm.append((what, e0, e1))

    def _staging_buffers(self, dev, need: int) -> dict:
        """`slots` pairs of fp32 device buffers of `chunk` elements, the copy
        streams (default priority) and the per-slot events, made once."""
        st = self._staging
        if st is None or st["bufs"][0][0].numel() < need:
            n = max(need, 1)
            st = self._staging = {
                "bufs": [(torch.empty(n, dtype=torch.float32, device=dev), torch.empty(n, dtype=torch.float32, device=dev)) for _ in range(self.slots)],
                "h2d": torch.cuda.Stream(dev),
                "d2h": torch.cuda.Stream(dev),
                "ev_in": [torch.cuda.Event() for _ in range(self.slots)],
                "ev_done": [torch.cuda.Event() for _ in range(self.slots)],
                "ev_back": [torch.cuda.Event() for _ in range(self.slots)],
                "used": [False] * self.slots,
            }
        return st

    def promote(self, budget_bytes: int) -> int:
        """runtime/optim.py:208-227: move the host moments of parameters, in
        order, onto the GPU while they fit `budget_bytes` (8 bytes per
        element); the update reads and writes the same values wherever they
        live, so no bit changes.  -> bytes moved (0 for device moments)."""
        if self.moments != "host":
            return 0
        moved = 0
        for i, p in enumerate(self.params):
            if i in self.resident or not p.requires_grad or p.device.type != "cuda":
                continue
            need = 8 * p.numel()
            if moved + need > budget_bytes:
                continue
            st = self._slot(i, p)
            st["exp_avg"] = st["exp_avg"].to(p.device)
            st["exp_avg_sq"] = st["exp_avg_sq"].to(p.device)
            self.resident.add(i)
            moved += need
        if moved:
            torch.cuda.synchronize()
        return moved

    def _clip_coef(self, grads, accs=None, garr=None) -> int:
        """Launch the deterministic norm of every gradient of the step (any
        dtype; with accs, of the folded sums); returns the device address of
        its fp32 clip coefficient.  garr: the gradients' table, if built."""
        L = _lib.load()
        dev = grads[0].device
        if self._norm is None or self._norm.device != dev:
            self._norm = torch.empty(16, dtype=torch.uint8, device=dev)
        if garr is None:
            garr = _lib.tensor_array(grads)
        ws = _lib.workspace(dev, L.ely_grad_norm_workspace_bytes(garr, len(grads)))
        if accs is None:
            rc = L.ely_grad_norm(garr, len(grads), self.max_norm, self._norm.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
        else:
            rc = L.ely_grad_norm_fold(_lib.tensor_array(accs), garr, len(grads), self.max_norm, self._norm.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
        _lib.check(rc, "grad norm")
        return self._norm.data_ptr() + 12

    def _launch(self, ps, gs, ms, vs, cs, consts, coef_ptr, accs, wd: bool) -> None:
        copies = [(_lib.ely_tensor(c) if c is not None else _lib.ElyTensor(None, 0, _lib.BF16, 0)) for c in cs]
        self._launch_arrays(len(ps), _lib.tensor_array(ps), _lib.tensor_array(gs), _lib.tensor_array(ms),
                            _lib.tensor_array(vs), _lib.tensor_array(copies), consts, coef_ptr,
                            None if accs is None else _lib.tensor_array(accs), ps[0].device, wd)

    def _launch_arrays(self, n, parr, garr, marr, varr, carr, consts, coef_ptr, aarr, dev, wd: bool) -> None:
        L = _lib.load()
        stream = _lib.stream_ptr(dev)
        if all(c is consts[0] for c in consts):
            # every tensor at one step: one row, repeated
            ctab = np.zeros((n, 8), dtype=np.float32)
            ctab[:, : len(consts[0])] = np.asarray(consts[0], dtype=np.float32)
        else:
            ctab = np.asarray(consts, dtype=np.float32).reshape(n, -1)
            if ctab.shape[1] < 8:
                ctab = np.pad(ctab, ((0, 0), (0, 8 - ctab.shape[1])))
            ctab = np.ascontiguousarray(ctab)
        carr_c = (_lib.ElyConsts * n).from_buffer(ctab)
        ws = _lib.workspace(dev, L.ely_adamw_workspace_bytes(n))
        order = _lib.ORDER_HOST if self.order == "host" else _lib.ORDER_TORCH
        wd = int(wd)
        if aarr is None:
            rc = L.ely_adamw_step(parr, garr, marr, varr, carr, n, carr_c, order, wd, coef_ptr, ws.data_ptr(), ws.numel(), stream)
        else:
            rc = L.ely_adamw_fold_step(parr, aarr, garr, marr, varr, carr, n, carr_c, order, wd, coef_ptr, ws.data_ptr(),
                                       ws.numel(), stream)
        _lib.check(rc, f"{self.recipe} step")

    def grad_norm(self) -> torch.Tensor | None:
        """The fp32 global gradient norm of the last clipped step (a device
        tensor, no synchronization), or None."""
        if self._norm is None:
            return None
        return self._norm[8:12].view(torch.float32).reshape(())

    def zero_grad(self, set_to_none: bool = True) -> None:
        for p in self.params:
            if set_to_none:
                p.grad = None
            elif p.grad is not None:
                p.grad.zero_()

    # --------------------------------------------------------- checkpoint

    def state_dict(self) -> dict:
        """torch's AdamW layout, keyed by parameter index; adamw-host returns
        host copies of the moments as the reference does
        (runtime/optim.py:238-250), "adamw" the moment tensors themselves as
        torch does.  The group is the live param group (a scheduler's lr
        included)."""
        host = self.order == "host"
        group = {k: v for k, v in self.param_groups[0].items() if k != "params"}
        return {
            "state": {
                i: {
                    "step": st["step"].clone(),
                    "exp_avg": st["exp_avg"].cpu() if host else st["exp_avg"],
                    "exp_avg_sq": st["exp_avg_sq"].cpu() if host else st["exp_avg_sq"],
                }
                for i, st in sorted(self._st.items())
            },
            "param_groups": [{**group, "params": list(range(len(self.params)))}],
        }

    def load_state_dict(self, sd: dict) -> None:
        """adamw-host: runtime/optim.py:252-274, refusing another recipe's
        state (any hyperparameter that differs), other parameters and wrong
        shapes.  adamw: torch.optim.Optimizer.load_state_dict's semantics
        (TORCH/optim/optimizer.py:877-1016): one group of as many parameters,
        whose saved hyperparameters (lr, betas, eps, weight_decay, and keys
        this build does not read) are adopted; amsgrad and maximize, which
        the fused kernel does not implement, are refused.  Parameters the
        state does not name start again from zero moments."""
        groups = sd.get("param_groups") or []
        if self.order == "torch":
            if len(groups) != 1:
                raise ValueError("loaded state dict has a different number of parameter groups")
            if len(groups[0]["params"]) != len(self.params):
                raise ValueError("loaded state dict contains a parameter group that doesn't match the size of optimizer's group")
            theirs = {k: v for k, v in groups[0].items() if k != "params"}
            for flag in ("amsgrad", "maximize"):
                if theirs.get(flag):
                    raise ValueError(f"{self.recipe} on MI355X steps AdamW without {flag}; the state asks for it")
            b1, b2 = theirs.get("betas", self.betas)
            self.lr = float(theirs.get("lr", self.lr))
            self.betas = (float(b1), float(b2))
            self.eps = float(theirs.get("eps", self.eps))
            self.weight_decay = float(theirs.get("weight_decay", self.weight_decay))
            self._group = {**self._group, **theirs}
            self.param_groups = [{**self._group, "params": self.params}]
            # the saved list of parameter ids maps onto this optimizer's, in order
            ids = {k: i for i, k in enumerate(groups[0]["params"])}
        else:
            if len(groups) != 1:
                raise ValueError(f"{self.recipe} state holds one param group")
            theirs = {k: v for k, v in groups[0].items() if k != "params"}
            mine = json_norm(self._group)
            if json_norm(theirs) != mine:
                raise ValueError(f"optimizer state of another recipe: {json_norm(theirs)} is not {mine}")
            if list(groups[0]["params"]) != list(range(len(self.params))):
                raise ValueError("optimizer state names other parameters")
            ids = {i: i for i in range(len(self.params))}
        states = {}
        for k, st in sd.get("state", {}).items():
            k = int(k) if isinstance(k, str) else k  # keys read back from JSON
            if k not in ids:
                raise ValueError("optimizer state names other parameters")
            i = ids[k]
            p = self.params[i]
            for name in ("exp_avg", "exp_avg_sq"):
                if tuple(st[name].shape) != tuple(p.shape):
                    raise ValueError(f"optimizer state {i}.{name} has shape {tuple(st[name].shape)}")
            states[i] = st
        self._st.clear()
        if self._flat_m is not None:
            self._steps.zero_()
        for i, st in sorted(states.items()):
            self._assign(i, st)


class HostAdamW(FusedAdamW):
    """The "adamw-host" recipe under the reference's class name
    (runtime/optim.py:77-298) and with its constructor's arguments:
    HostAdamW's op order, moments in pinned host memory.  The reference's
    runtime tests isinstance(opt, optim.HostAdamW) before promoting moments
    (runtime/stage.py:3134); build("adamw-host") returns this class, so that
    test holds for this build's optimizer.  FusedAdamW's other options
    (max_norm, working_copy, release_elems, moments="device") pass by
    keyword.  pipeline=None updates the moments in place through the GPU's
    mapping (this build's default); True and False are the reference's
    staged and serial copies."""

    def __init__(
        self,
        params: Iterable[torch.Tensor],
        lr: float,
        betas: tuple = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 0.0,
        chunk: int = CHUNK,
        pipeline: bool | None = None,
        slots: int = 3,
        **kw,
    ):
        kw.setdefault("moments", "host")
        super().__init__(params, lr, betas, eps, weight_decay, order="host", chunk=chunk, pipeline=pipeline,
                         slots=slots, **kw)


def clip_grad_norm_(parameters, max_norm: float, norm_type: float = 2.0, error_if_nonfinite: bool = False, foreach=None) -> torch.Tensor:
    """torch.nn.utils.clip_grad_norm_ (TORCH/nn/utils/clip_grad.py:50-183)
    for the 2-norm: the deterministic device norm of every gradient, then each
    gradient scaled in place by min(max_norm / (norm + 1e-6), 1).  Returns the
    fp32 total norm as a device tensor."""
    if norm_type != 2.0:
        raise ValueError("clip_grad_norm_ on MI355X computes the 2-norm only")
    if isinstance(parameters, torch.Tensor):
        parameters = [parameters]
    grads = [p.grad for p in parameters if p.grad is not None]
    if not grads:
        return torch.tensor(0.0)
    dev = grads[0].device
    for g in grads:
        _lib.require_gpu(g, "clip_grad_norm_")
        if g.device != dev or not g.is_contiguous():
            raise ValueError("clip_grad_norm_: gradients must be contiguous and on one device")
    L = _lib.load()
    with torch.cuda.device(dev):
        res = torch.empty(16, dtype=torch.uint8, device=dev)
        garr = _lib.tensor_array(grads)
        ws = _lib.workspace(dev, L.ely_grad_norm_workspace_bytes(garr, len(grads)))
        sp = _lib.stream_ptr(dev)
        if not error_if_nonfinite:
            # the norm, then g <- g * coef in g's dtype over every gradient in one launch
            _lib.check(L.ely_grad_norm_clip(garr, len(grads), float(max_norm), res.data_ptr(), ws.data_ptr(), ws.numel(), sp), "clip_grad_norm_")
            return res[8:12].view(torch.float32).reshape(()).clone()
        _lib.check(L.ely_grad_norm(garr, len(grads), float(max_norm), res.data_ptr(), ws.data_ptr(), ws.numel(), sp), "clip_grad_norm_")
        total = res[8:12].view(torch.float32).reshape(()).clone()
        if bool(~torch.isfinite(total)):
            raise RuntimeError(f"The total norm of order {norm_type} for gradients from `parameters` is non-finite, so it cannot be clipped.")
        # g <- g * coef in g's dtype, torch's _foreach_mul_ by the clamped coefficient
        _lib.check(L.ely_scale_inplace(garr, len(grads), res.data_ptr() + 12, sp), "clip_grad_norm_ scale")
    return total
