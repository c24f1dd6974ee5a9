"""Bit fingerprints of tensors for the recompute check (reference: recompute.py:59-116, _fingerprint.py).

fingerprint(t) -> int64[3] on t's device: the sums of t's 16-bit words (8-bit for 1-byte dtypes), and of the words
times two pseudo-random odd 64-bit weights of their position (splitmix64's mix of position + 0x9E3779B97F4A7C15),
mod 2^64.  One HIP kernel pass (sdc_fingerprint3), bit-exact: wrapping integer sums do not depend on order.
"""
from __future__ import annotations

import torch

from . import _lib

# recompute.py:59-61, as signed int64 (0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9, 0x94D049BB133111EB)
_FP_SEED = -7046029254386353131
_FP_M1 = -4658895280553007687
_FP_M2 = -7723592293110705685


def fingerprint_bits(bits: torch.Tensor, start: int = 0, out: torch.Tensor = None) -> torch.Tensor:
    """The three sums of a flat int16 or int8 tensor (recompute.py:72-90's fast path, _fingerprint.py:128-130).
    With `out` ([3] int64 on the device) the sums are added into it."""
    if bits.dtype not in (torch.int16, torch.int8) or bits.dim() != 1 or not bits.is_contiguous():
        raise ValueError("fingerprint_bits takes a flat contiguous int16 or int8 tensor")
    _lib.require_gpu(bits)
    if out is None:
        out = torch.zeros(3, dtype=torch.int64, device=bits.device)
    rc = _lib.lib().sdc_fingerprint3(bits.data_ptr(), bits.numel(), bits.element_size(), int(start), out.data_ptr(),
                                     _lib.stream_of(bits))
    _lib.check(rc, "sdc_fingerprint3")
    return out


def fingerprint(t: torch.Tensor) -> torch.Tensor:
    """recompute.py:72-90: [3] int64 on t's device, no host sync."""
    x = t.detach()
    if x.numel() == 0:
        return torch.zeros(3, dtype=torch.int64, device=x.device)
    x = x.contiguous().view(-1)
    bits = x.view(torch.int16) if x.element_size() % 2 == 0 else x.view(torch.int8)
    return fingerprint_bits(bits)


# ---------------------------------------------------------------------------------------------------------------
# The exact recompute check (the reference's RecomputeCheck, recompute.py:148-450; built here on a device ledger)
#
# Activation checkpointing runs each checkpointed block twice: in the forward pass, and again in the backward pass to
# rebuild the activations it did not keep.  With deterministic kernels on a healthy GPU both runs give the same bits.
# Each output of a block gets a row of a per-device ledger, int64 [rows, 2, 3]: the forward run's fingerprint is
# added into [row, 0], the recompute's into [row, 1] (sdc_fingerprint3 adds into its output, so nothing is allocated
# per output).  flush() compares all rows of a device in one operation and reads one flag per row back.  No noise
# model and no threshold; it sees any operation inside a block.  It cannot see a fault that gives the same wrong bits
# both times, blocks that are not checkpointed, or blocks checkpointed without preserving the RNG state (skipped and
# counted); nondeterministic kernels show as mismatches (calibrate() says whether clean recomputes match).

import contextlib
import functools
import sys
import threading
import weakref
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional


def _tensors_in(out) -> list:
    """The tensors a block returned, in a fixed order: depth first through tuples and lists, dicts by sorted key."""
    if isinstance(out, torch.Tensor):
        return [out]
    if isinstance(out, (tuple, list)):
        return [t for o in out for t in _tensors_in(o)]
    if isinstance(out, dict):
        return [t for k in sorted(out, key=str) for t in _tensors_in(out[k])]
    return []


def _block_name(function) -> str:
    """A block's name for reports: the module class (and method) behind a callable, through partials."""
    while isinstance(function, functools.partial):
        function = function.func
    if isinstance(function, torch.nn.Module):
        return type(function).__name__
    bound_to = getattr(function, "__self__", None)
    if isinstance(bound_to, torch.nn.Module):
        return f"{type(bound_to).__name__}.{getattr(function, '__name__', 'forward')}"
    return getattr(function, "__qualname__", None) or type(function).__name__


class _Router:
    """Where torch's checkpoint function is replaced by the dispatcher while at least one check is installed: the
    torch.utils.checkpoint attribute, every module attribute that imported it by another name, and the checkpoint
    partials held by the modules of attached models.  Everything is put back when the last check leaves."""

    def __init__(self):
        self.lock = threading.RLock()
        self.original = None
        self.checks: list = []                 # installed, newest last (the newest records)
        self.names: list = []                  # (module, attribute) now holding the dispatcher
        self.partials: list = []               # (module object, attribute, old partial, new partial)

    def torch_checkpoint(self):
        if self.original is None:
            import torch.utils.checkpoint as tuc
            if tuc.checkpoint is not dispatch:
                self.original = tuc.checkpoint
        return self.original

    def enter(self, check) -> None:
        import torch.utils.checkpoint as tuc
        orig = self.torch_checkpoint()
        if not self.checks and tuc.checkpoint is orig:
            tuc.checkpoint = dispatch
            for mod in list(sys.modules.values()):
                d = getattr(mod, "__dict__", None)
                if not isinstance(d, dict) or mod is tuc or d.get("dispatch") is dispatch:
                    continue
                for attr in [a for a, v in list(d.items()) if v is orig]:
                    setattr(mod, attr, dispatch)
                    self.names.append((mod, attr))
        self.checks.append(check)

    def reroute(self, model: torch.nn.Module) -> None:
        orig = self.torch_checkpoint()
        for mod in model.modules():
            for attr, val in list(vars(mod).items()):
                if isinstance(val, functools.partial) and val.func is orig:
                    new = functools.partial(dispatch, *val.args, **(val.keywords or {}))
                    mod.__dict__[attr] = new
                    self.partials.append((mod, attr, val, new))

    def leave(self, check) -> None:
        import torch.utils.checkpoint as tuc
        self.checks.remove(check)
        if self.checks:
            return
        orig = self.torch_checkpoint()
        if tuc.checkpoint is dispatch:
            tuc.checkpoint = orig
        for mod, attr in self.names:
            if getattr(mod, attr, None) is dispatch:
                setattr(mod, attr, orig)
        for mod, attr, old, new in self.partials:
            if mod.__dict__.get(attr) is new:
                mod.__dict__[attr] = old
        self.names.clear()
        self.partials.clear()


_ROUTER = _Router()


def dispatch(function=None, *args, **kwargs):
    """What torch.utils.checkpoint.checkpoint is while a RecomputeCheck is installed (after the last uninstall, a
    reference to it kept somewhere runs torch's own)."""
    with _ROUTER.lock:
        check = _ROUTER.checks[-1] if _ROUTER.checks else None
    if check is None:
        return _ROUTER.torch_checkpoint()(function, *args, **kwargs)
    return check.checkpoint(function, *args, **kwargs)


_dispatch = dispatch                 # (the name callers and tests have used)


@dataclass
class _Run:
    """One checkpointed block call: its outputs' ledger rows (first .. first + n - 1) and how far it got."""
    name: str
    call: int
    device: Optional[torch.device] = None
    first: int = -1
    n: int = 0
    runs: int = 0                     # 1: forward fingerprinted; 2: recompute fingerprinted too


class _Ledger:
    """One device's rows of [forward, recompute] fingerprints (int64 [rows, 2, 3]), handed out in order and cleared
    at each flush."""

    def __init__(self, device: torch.device, rows: int):
        with torch.inference_mode(False):
            self.t = torch.zeros(rows, 2, 3, dtype=torch.int64, device=device)
        self.used = 0

    def take(self, n: int) -> int:
        """First of n free rows, or -1 when the ledger is full."""
        if self.used + n > self.t.shape[0]:
            return -1
        self.used += n
        return self.used - n

    def add(self, row: int, run: int, t: torch.Tensor) -> None:
        x = t.detach()
        if x.numel() == 0:
            return
        x = x.contiguous().view(-1)
        bits = x.view(torch.int16) if x.element_size() % 2 == 0 else x.view(torch.int8)
        fingerprint_bits(bits, out=self.t[row, run])

    def differing(self) -> List[bool]:
        """Per used row, whether the two fingerprints differ (one read-back); then every row is cleared."""
        if not self.used:
            return []
        flags = (self.t[:self.used, 0] != self.t[:self.used, 1]).any(-1).cpu().tolist()
        self.t[:self.used].zero_()
        self.used = 0
        return flags


class RecomputeCheck:
    """Compares each checkpointed block's forward outputs with its recompute, bit for bit, through fingerprints.
    install() routes torch's checkpoint through it; flush() compares what ran since the last flush."""

    def __init__(self, on_alert: Optional[Callable] = None, max_pending: int = 8192):
        self.on_alert = on_alert
        self.max_pending = int(max_pending)        # ledger rows per device (block outputs awaiting a flush)
        self.step: Optional[int] = None
        self.enabled = True
        self.events: list = []
        self.stats = {"blocks_run": 0, "recomputes_compared": 0, "mismatches": 0, "never_recomputed": 0,
                      "dropped_queue_full": 0, "skipped_rng_not_preserved": 0, "selective_blocks": 0}
        self._models: list = []                    # weak references to attached models
        self._runs: Dict[int, _Run] = {}
        self._ledgers: Dict[torch.device, _Ledger] = {}
        self._calls = 0
        self._installed = False
        self._lock = threading.RLock()

    # -------------------------------------------------------------------------------------------------- routing
    def install(self, model: Optional[torch.nn.Module] = None) -> "RecomputeCheck":
        """Route torch.utils.checkpoint.checkpoint (and the names other modules imported it under; with a model, the
        checkpoint partials its modules hold) through this check until uninstall()."""
        with _ROUTER.lock:
            if model is not None:
                self.attach(model)
            if not self._installed:
                _ROUTER.enter(self)
                self._installed = True
                for ref in list(self._models):
                    m = ref()
                    if m is not None:
                        _ROUTER.reroute(m)
        return self

    def attach(self, model: torch.nn.Module) -> "RecomputeCheck":
        with _ROUTER.lock:
            self._models = [r for r in self._models if r() is not None]
            if all(r() is not model for r in self._models):
                self._models.append(weakref.ref(model))
            if self._installed:
                _ROUTER.reroute(model)
        return self

    def uninstall(self) -> None:
        with _ROUTER.lock:
            if self._installed:
                self._installed = False
                _ROUTER.leave(self)

    def __enter__(self):
        return self.install()

    def __exit__(self, *exc):
        self.uninstall()
        return False

    # ---------------------------------------------------------------------------------------------- the blocks
    def checkpoint(self, function, *args, **kwargs):
        """torch.utils.checkpoint.checkpoint, with the block's two runs fingerprinted into the ledger."""
        orig = _ROUTER.torch_checkpoint()
        if function is None or not self.enabled:
            return orig(function, *args, **kwargs)
        if kwargs.get("preserve_rng_state", True) is False:          # its dropout masks differ by design
            with self._lock:
                self.stats["skipped_rng_not_preserved"] += 1
            return orig(function, *args, **kwargs)
        with self._lock:
            if kwargs.get("context_fn") not in (None, getattr(torch.utils.checkpoint, "noop_context_fn", None)):
                self.stats["selective_blocks"] += 1
            self._calls += 1
            run = self._runs[self._calls] = _Run(_block_name(function), self._calls)
            self.stats["blocks_run"] += 1

        def fingerprinted(*a, **k):
            out = function(*a, **k)
            try:
                with torch.no_grad():
                    self._record(run, _tensors_in(out))
            except Exception:  # noqa: BLE001  (an output the fingerprint cannot take never breaks training)
                pass
            return out

        # the recompute must run the whole block, so that every output exists to compare
        early = getattr(torch.utils.checkpoint, "set_checkpoint_early_stop", None)
        with (early(False) if early is not None else contextlib.nullcontext()):
            return orig(fingerprinted, *args, **kwargs)

    def _record(self, run: _Run, outs: list) -> None:
        with self._lock:
            if run.runs == 0:
                run.runs = 1
                if not outs:
                    return
                dev = outs[0].device
                led = self._ledgers.get(dev)
                if led is None:
                    led = self._ledgers[dev] = _Ledger(dev, self.max_pending)
                first = led.take(len(outs))
                if first < 0:
                    self.stats["dropped_queue_full"] += 1
                    self._runs.pop(run.call, None)
                    return
                run.device, run.first, run.n = dev, first, len(outs)
                which = 0
            elif run.runs == 1 and run.first >= 0 and len(outs) == run.n:
                run.runs = 2
                which = 1
            else:
                return
            led = self._ledgers[run.device]
            for j, t in enumerate(outs):
                led.add(run.first + j, which, t.to(run.device) if t.device != run.device else t)

    # -------------------------------------------------------------------------------------------------- results
    def flush(self) -> list:
        """Compare every block recomputed since the last flush (one comparison and one read-back per device) and
        report the mismatches; blocks never recomputed are counted and dropped."""
        from .serve import SDCEvent
        with self._lock:
            runs, self._runs = list(self._runs.values()), {}
            ledgers = dict(self._ledgers)
            flags = {dev: led.differing() for dev, led in ledgers.items()}
        events = []
        for run in runs:
            if run.runs < 2 or run.first < 0:
                self.stats["never_recomputed"] += run.runs == 1 or run.first < 0
                continue
            self.stats["recomputes_compared"] += 1
            bad = [j for j in range(run.n) if flags[run.device][run.first + j]]
            if not bad:
                continue
            self.stats["mismatches"] += 1
            ev = SDCEvent(detector="recompute", layer=run.name, z=float("inf"),
                          extra={"where": run.name, "block_call": run.call, "outputs_that_differ": bad,
                                 "step": self.step,
                                 "reading": "this checkpointed block gave other bits when the backward pass recomputed "
                                            "it: an operation inside it computed another result the second time; on a "
                                            "healthy GPU with deterministic kernels both runs match exactly "
                                            "(calibrate() says whether they do)"})
            events.append(ev)
            self.events.append(ev)
        failure = None
        for ev in events:
            if self.on_alert is not None:
                try:
                    self.on_alert(ev)
                except Exception as e:  # noqa: BLE001  (every callback runs; the first failure is raised after)
                    failure = failure or e
        if failure is not None:
            raise failure
        return events

    def calibrate(self, step_fn: Callable[[], None], steps: int = 3) -> dict:
        """Run step_fn (a forward and backward with checkpointing) a few times on a healthy GPU: whether every
        recompute was bit-identical (mismatches here come from nondeterministic kernels, not faults)."""
        before = self.stats["recomputes_compared"]
        seen: list = []
        kept, self.on_alert = self.on_alert, seen.append
        try:
            with self:
                for _ in range(steps):
                    step_fn()
                    self.flush()
        finally:
            self.on_alert = kept
        n = self.stats["recomputes_compared"] - before
        return {"recomputes_compared": n, "mismatches": len(seen),
                "blocks_that_differed": sorted({ev.extra["where"] for ev in seen}),
                "deterministic": n > 0 and not seen,
                "note": None if n else "no recompute ran: is gradient checkpointing on, and did step_fn call "
                                       "backward()?"}

    def coverage(self, model: torch.nn.Module, step_fn: Callable[[], None]) -> dict:
        """Run step_fn once: how many blocks were compared, and the share of the model's parameters held by modules
        that ran inside a compared block."""
        inside: set = set()
        depth = [0]

        def note(mod, inp, out):
            if depth[0]:
                inside.add(id(mod))

        class _Counting:
            """The check with each block's function wrapped to count its depth."""
            def __init__(self, check):
                self.check = check

            def checkpoint(self, function, *a, **k):
                def deep(*x, **y):
                    depth[0] += 1
                    try:
                        return function(*x, **y)
                    finally:
                        depth[0] -= 1
                return self.check.checkpoint(deep, *a, **k)

        hook = torch.nn.modules.module.register_module_forward_hook(note)
        before = dict(self.stats)
        was_installed, was_enabled = self._installed, self.enabled
        counting = _Counting(self)
        self.enabled = True
        try:
            self.install(model)
            with _ROUTER.lock:
                _ROUTER.checks.append(counting)
            try:
                step_fn()
            finally:
                with _ROUTER.lock:
                    _ROUTER.checks.remove(counting)
            self.flush()
        finally:
            self.enabled = was_enabled
            hook.remove()
            if not was_installed:
                self.uninstall()
        total = sum(p.numel() for p in model.parameters())
        covered = sum(p.numel() for mod in model.modules() if id(mod) in inside for p in mod.parameters(recurse=False))
        outside = sorted({type(mod).__name__ for mod in model.modules()
                          if next(mod.parameters(recurse=False), None) is not None and id(mod) not in inside})
        return {"blocks_compared": self.stats["recomputes_compared"] - before["recomputes_compared"],
                "blocks_skipped_rng": self.stats["skipped_rng_not_preserved"] - before["skipped_rng_not_preserved"],
                "parameter_share_inside_compared_blocks": round(covered / total, 4) if total else 0.0,
                "module_types_with_parameters_outside": outside[:20]}
