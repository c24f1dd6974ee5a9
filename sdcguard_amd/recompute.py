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
# The exact recompute check (recompute.py:148-450)
#
# Activation checkpointing runs each checkpointed block twice: in the forward pass and again in the backward pass
# to rebuild the activations it didn't keep.  With deterministic kernels on a healthy GPU the two runs give the same
# bits, so every output of the first run is fingerprinted, the same outputs of the recompute too, and a flush
# compares them (one comparison and one read-back per device for all the step's blocks).  No noise model, no
# threshold; it covers any operation inside a block.  It can't see a fault that repeats the same wrong bits both
# times, blocks that aren't checkpointed, or blocks checkpointed without preserving the RNG state (skipped and
# counted); nondeterministic kernels report as mismatches (calibrate() says whether clean recomputes match).

import contextlib
import functools
import sys
import threading
import weakref
from typing import Callable, Optional

_LOCK = threading.RLock()
_CHECKPOINT = [None]            # torch's checkpoint, kept once the check is first installed
_PATCHED: list = []             # (module, attribute) that held torch's checkpoint and now hold _dispatch
_PARTIALS: list = []            # (module, attribute, old partial, new partial) rerouted on attached models
_INSTALLED: list = []           # RecomputeCheck objects installed (the newest records)


def _torch_checkpoint():
    if _CHECKPOINT[0] is None:
        import torch.utils.checkpoint as tuc
        _CHECKPOINT[0] = tuc.checkpoint if tuc.checkpoint is not _dispatch else None
    return _CHECKPOINT[0]


def _outputs(out) -> list:
    """The tensors a block returned (nested tuples, lists and dicts, dict keys in sorted order)."""
    found = []
    stack = [out]
    while stack:
        o = stack.pop()
        if isinstance(o, torch.Tensor):
            found.append(o)
        elif isinstance(o, (tuple, list)):
            stack.extend(reversed(o))
        elif isinstance(o, dict):
            stack.extend(o[k] for k in sorted(o, key=str, reverse=True))
    return found


def _name(function) -> str:
    f = function
    while isinstance(f, functools.partial):
        f = f.func
    owner = getattr(f, "__self__", None)
    if isinstance(owner, torch.nn.Module):
        return type(owner).__name__ + "." + getattr(f, "__name__", "forward")
    if isinstance(f, torch.nn.Module):
        return type(f).__name__
    return getattr(f, "__qualname__", None) or type(f).__name__


class RecomputeCheck:
    """Compares each checkpointed block's forward outputs with its recompute through their fingerprints."""

    def __init__(self, on_alert: Optional[Callable] = None, max_pending: int = 8192):
        self.on_alert = on_alert
        self.max_pending = int(max_pending)
        self.step: Optional[int] = None
        self.enabled = True
        self.events: list = []
        self.stats = {"blocks_run": 0, "recomputes_compared": 0, "mismatches": 0, "never_recomputed": 0,
                      "dropped_queue_full": 0, "skipped_rng_not_preserved": 0, "selective_blocks": 0}
        self._models: list = []          # weak references to models whose stored checkpoint partials are rerouted
        self._open: dict = {}            # call index -> (name, forward fingerprints)
        self._pending: list = []         # (name, call index, forward fingerprints, recompute fingerprints)
        self._calls = 0
        self._installed = False

    # ------------------------------------------------------------------------------------------- routing
    def install(self, model: Optional[torch.nn.Module] = None) -> "RecomputeCheck":
        """Route torch.utils.checkpoint.checkpoint (and the names other modules imported it under, and with a model
        the checkpoint partials its modules hold) through this check.  uninstall() puts them back."""
        import torch.utils.checkpoint as tuc
        with _LOCK:
            if model is not None:
                self.attach(model)
            if self._installed:
                return self
            orig = _torch_checkpoint()
            if tuc.checkpoint is orig:
                tuc.checkpoint = _dispatch
                for mod in list(sys.modules.values()):
                    d = getattr(mod, "__dict__", None)
                    if not isinstance(d, dict) or mod is tuc or d.get("_dispatch") is _dispatch:
                        continue
                    for attr, val in list(d.items()):
                        if val is orig:
                            setattr(mod, attr, _dispatch)
                            _PATCHED.append((mod, attr))
            _INSTALLED.append(self)
            self._installed = True
            self._reroute()
        return self

    def attach(self, model: torch.nn.Module) -> "RecomputeCheck":
        with _LOCK:
            if not any(r() is model for r in self._models):
                self._models.append(weakref.ref(model))
            if self._installed:
                self._reroute()
        return self

    def _reroute(self) -> None:
        orig = _torch_checkpoint()
        for ref in list(self._models):
            m = ref()
            if m is None:
                self._models.remove(ref)
                continue
            for mod in m.modules():
                for attr, val in list(vars(mod).items()):
                    if isinstance(val, functools.partial) and val.func is orig:
                        new = functools.partial(_dispatch, *val.args, **(val.keywords or {}))
                        mod.__dict__[attr] = new
                        _PARTIALS.append((mod, attr, val, new))

    def uninstall(self) -> None:
        import torch.utils.checkpoint as tuc
        with _LOCK:
            if not self._installed:
                return
            _INSTALLED.remove(self)
            self._installed = False
            if _INSTALLED:
                return
            orig = _torch_checkpoint()
            if tuc.checkpoint is _dispatch:
                tuc.checkpoint = orig
            for mod, attr in _PATCHED:
                if getattr(mod, attr, None) is _dispatch:
                    setattr(mod, attr, orig)
            _PATCHED.clear()
            for mod, attr, old, new in _PARTIALS:
                if mod.__dict__.get(attr) is new:
                    mod.__dict__[attr] = old
            _PARTIALS.clear()

    def __enter__(self):
        return self.install()

    def __exit__(self, *exc):
        self.uninstall()
        return False

    # ------------------------------------------------------------------------------------------- the block
    def checkpoint(self, function, *args, **kwargs):
        """torch.utils.checkpoint.checkpoint that also compares the recompute with the forward run."""
        orig = _torch_checkpoint()
        if function is None or not self.enabled:
            return orig(function, *args, **kwargs)
        if kwargs.get("preserve_rng_state", True) is False:      # dropout masks differ by design
            with _LOCK:
                self.stats["skipped_rng_not_preserved"] += 1
            return orig(function, *args, **kwargs)
        if kwargs.get("context_fn") not in (None, getattr(torch.utils.checkpoint, "noop_context_fn", None)):
            with _LOCK:
                self.stats["selective_blocks"] += 1
        with _LOCK:
            self._calls += 1
            idx = self._calls
            self.stats["blocks_run"] += 1
        name = _name(function)
        runs = [0]

        def wrapped(*a, **k):
            out = function(*a, **k)
            try:
                with torch.no_grad():
                    fps = [fingerprint(t) for t in _outputs(out)]
            except Exception:  # noqa: BLE001  (an output the fingerprint can't take never breaks training)
                return out
            runs[0] += 1
            with _LOCK:
                if runs[0] == 1:
                    if len(self._open) >= self.max_pending:        # never recomputed (no backward): drop the oldest
                        self._open.pop(next(iter(self._open)))
                        self.stats["never_recomputed"] += 1
                    self._open[idx] = (name, fps)
                else:
                    first = self._open.pop(idx, None)
                    if first is not None and len(first[1]) == len(fps):
                        if len(self._pending) >= self.max_pending:
                            self.stats["dropped_queue_full"] += 1
                        else:
                            self._pending.append((first[0], idx, first[1], fps))
            return out

        # the recompute must run the whole block so its outputs exist to compare
        early = getattr(torch.utils.checkpoint, "set_checkpoint_early_stop", None)
        with (early(False) if early is not None else contextlib.nullcontext()):
            return orig(wrapped, *args, **kwargs)

    # ------------------------------------------------------------------------------------------- results
    def flush(self) -> list:
        """Compare every recompute queued since the last flush (one comparison and one read-back per device) and
        report mismatches; blocks never recomputed are counted and dropped."""
        from .serve import SDCEvent
        with _LOCK:
            pending, self._pending = self._pending, []
            self.stats["never_recomputed"] += len(self._open)
            self._open = {}
        if not pending:
            return []
        by_dev: dict = {}
        for i, (_, _, first, _) in enumerate(pending):
            if first:
                by_dev.setdefault(first[0].device, []).append(i)
        bad_outputs: dict = {}
        for dev, idxs in by_dev.items():
            a = torch.stack([f.to(dev) for i in idxs for f in pending[i][2]])
            b = torch.stack([f.to(dev) for i in idxs for f in pending[i][3]])
            differ = (a != b).any(-1).cpu().tolist()
            pos = 0
            for i in idxs:
                k = len(pending[i][2])
                bad_outputs[i] = [j for j, d in enumerate(differ[pos:pos + k]) if d]
                pos += k
        events = []
        for i, (name, idx, _, _) in enumerate(pending):
            self.stats["recomputes_compared"] += 1
            bad = bad_outputs.get(i) or []
            if not bad:
                continue
            self.stats["mismatches"] += 1
            ev = SDCEvent(detector="recompute", layer=name, z=float("inf"),
                          extra={"where": name, "block_call": idx, "outputs_that_differ": bad, "step": self.step,
                                 "reading": "this checkpointed block gave different bits when training recomputed "
                                            "it: an operation inside it computed a different result the second "
                                            "time; on a healthy GPU with deterministic kernels the two runs match "
                                            "exactly (calibrate() tells whether they do)"})
            events.append(ev)
            self.events.append(ev)
        err = None
        for ev in events:
            if self.on_alert is not None:
                try:
                    self.on_alert(ev)
                except Exception as e:  # noqa: BLE001
                    err = err or e
        if err is not None:
            raise err
        return events

    def calibrate(self, step_fn: Callable[[], None], steps: int = 3) -> dict:
        """Run step_fn (one forward and backward with checkpointing) a few times on a healthy GPU: whether every
        recompute was bit-identical (mismatches here are nondeterministic kernels, not faults)."""
        before = self.stats["recomputes_compared"]
        seen = []
        saved, self.on_alert = self.on_alert, seen.append
        try:
            with self:
                for _ in range(steps):
                    step_fn()
                    self.flush()
        finally:
            self.on_alert = saved
        compared = self.stats["recomputes_compared"] - before
        return {"recomputes_compared": compared, "mismatches": len(seen),
                "blocks_that_differed": sorted({ev.extra["where"] for ev in seen}),
                "deterministic": compared > 0 and not seen,
                "note": None if compared else "no recompute ran: is gradient checkpointing on, and did step_fn call "
                                              "backward()?"}

    def coverage(self, model: torch.nn.Module, step_fn: Callable[[], None]) -> dict:
        """Run step_fn once: how many blocks were compared and which share of the model's parameters belongs to
        modules that ran inside a compared block."""
        inside: set = set()
        depth = [0]

        def hook(mod, inp, out):
            if depth[0] > 0:
                inside.add(id(mod))
        h = torch.nn.modules.module.register_module_forward_hook(hook)
        plain = self.checkpoint

        def counting(function, *a, **k):
            def f(*x, **y):
                depth[0] += 1
                try:
                    return function(*x, **y)
                finally:
                    depth[0] -= 1
            return plain(f, *a, **k)
        before = dict(self.stats)
        was_installed, was_enabled = self._installed, self.enabled
        self.checkpoint = counting
        self.enabled = True
        try:
            self.install(model)
            step_fn()
            self.flush()
        finally:
            del self.checkpoint
            self.enabled = was_enabled
            h.remove()
            if not was_installed:
                self.uninstall()
        total = sum(p.numel() for p in model.parameters())
        covered = sum(p.numel() for mod in model.modules() if id(mod) in inside for p in mod.parameters(recurse=False))
        outside = sorted({type(mod).__name__ for mod in model.modules()
                          if any(True for _ in mod.parameters(recurse=False)) and id(mod) not in inside})
        return {"blocks_compared": self.stats["recomputes_compared"] - before["recomputes_compared"],
                "blocks_skipped_rng": self.stats["skipped_rng_not_preserved"] - before["skipped_rng_not_preserved"],
                "parameter_share_inside_compared_blocks": round(covered / total, 4) if total else 0.0,
                "module_types_with_parameters_outside": outside[:20]}


def _dispatch(function=None, *args, **kwargs):
    """What torch.utils.checkpoint.checkpoint is while a RecomputeCheck is installed."""
    with _LOCK:
        rc = _INSTALLED[-1] if _INSTALLED else None
    if rc is None:                       # a reference taken while installed, called after uninstall
        return _torch_checkpoint()(function, *args, **kwargs)
    return rc.checkpoint(function, *args, **kwargs)
