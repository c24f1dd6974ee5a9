"""Host side shared by the serving checks that run once per model step: the FP8 quantization check, the sampled
MoE recompute, the sampled attention recompute and the router check.

Each of them has kernels that fold what they find into one int64 state row per checked layer (atomic maxima of
packed keys, counters) and, for some, a kept record of the first sample over the alert line.  Around those rows the
host needs the same four things, which this module provides once:

  StepWord      the device word the kernels read to know which model step they run in: [step, armed, real rows,
                step | rows << 32] (the first two are the attention check's control pair).  mark_step() writes it
                with one asynchronous copy from a fresh pinned buffer (the caching host allocator keeps the buffer
                until the copy has run), so a guarded step never waits for the device; a graph captured once reads
                each replay's step from it.
  DeviceTable   per device, the state rows [rows, COLS] and the named capture tensors [rows, width], grown by
                doubling while layers are added (never after a graph has captured them: layers are added at load).
  Binding       what a layer's call site holds: the checks object and the layer's slot.  The tensors are looked up
                at each call, so a table that grew never leaves a layer writing rows nobody reads.
  StepChecks    registration, step marking, asynchronous read-back (a poll starts a copy into pinned memory and a
                later poll reports it; poll(wait=True) reports everything up to now), and the alert plumbing.  A
                subclass says what one state row means (_judge) and what its per-layer statistics are (_count).

No reference module has this split: the reference repeats the state / poll / report code in each check class
(serve_fp8.py:251-419, serve_moe.py:780-1051, serve_attn.py:890-1274).
"""
from __future__ import annotations

import struct
import threading
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

M32 = 0xFFFFFFFF
ROWS_SHIFT = 32
ROWS_MAX = (1 << 31) - 1

# the step word: what mark_step publishes on every device
W_STEP, W_ARMED, W_ROWS, W_PACKED = range(4)


def f32_of(bits: int) -> float:
    """The float whose bits are the low 32 bits of an int64 key."""
    return struct.unpack("<f", struct.pack("<I", int(bits) & M32))[0]


def pack_step(step: int, rows: Optional[int] = None) -> int:
    """step (low 32 bits) | real rows << 32 (0: not known)."""
    r = int(rows) if rows is not None and int(rows) > 0 else 0
    return (min(r, ROWS_MAX) << ROWS_SHIFT) | (int(step) & M32)


class StepWord:
    """int64[4] on one device: [step, armed (1 inside a marked step), real rows (0 unknown), step | rows << 32]."""

    def __init__(self, device: torch.device):
        with torch.inference_mode(False):
            self.t = torch.zeros(4, dtype=torch.int64, device=device)

    def write(self, step: int, rows: Optional[int], armed: bool) -> None:
        vals = [int(step) & M32, int(bool(armed)), int(rows) if rows else 0, pack_step(step, rows)]
        host = torch.tensor(vals, dtype=torch.int64)
        if self.t.is_cuda:
            host = host.pin_memory()
        self.t.copy_(host, non_blocking=self.t.is_cuda)

    def view(self, i: int, n: int = 1) -> torch.Tensor:
        return self.t[i:i + n]


class DeviceTable:
    """One device's state rows and capture tensors.  `capture` maps a name to (dtype, width)."""

    def __init__(self, device: torch.device, cols: int, rows: int, capture: Dict[str, Tuple[torch.dtype, int]]):
        self.device, self.cols = device, cols
        with torch.inference_mode(False):
            self.state = torch.zeros(rows, cols, dtype=torch.int64, device=device)
            self.capture = {k: torch.zeros(rows, max(int(w), 1), dtype=dt, device=device)
                            for k, (dt, w) in capture.items()}
        self.word = StepWord(device)

    @property
    def rows(self) -> int:
        return self.state.shape[0]

    def fit(self, rows: int, widths: Dict[str, int]) -> None:
        """Room for `rows` rows and at least `widths` columns of each capture tensor, keeping what is there."""
        grow_rows = rows > self.rows
        n = max(rows, 2 * self.rows) if grow_rows else self.rows
        with torch.inference_mode(False):
            if grow_rows:
                st = torch.zeros(n, self.cols, dtype=torch.int64, device=self.device)
                st[:self.rows] = self.state
                self.state = st
            for k, t in list(self.capture.items()):
                w = max(int(widths.get(k, 0)), t.shape[1])
                if grow_rows or w > t.shape[1]:
                    c = torch.zeros(n, w, dtype=t.dtype, device=self.device)
                    c[:t.shape[0], :t.shape[1]] = t
                    self.capture[k] = c


@dataclass(eq=False)
class Registered:
    """One checked layer."""
    name: str
    module: object
    device: torch.device
    slot: int                        # its row in the device's table
    info: dict = field(default_factory=dict)
    calls: int = 0                   # calls judged so far (from the state rows read back)
    worst: float = 0.0


@dataclass(eq=False)
class Binding:
    """What a layer's call site holds (layer._sdcguard_<check>): the checks object and the layer's slot."""
    checks: "StepChecks"
    slot: int

    @property
    def layer(self) -> Registered:
        return self.checks.layers[self.slot]

    def table(self) -> DeviceTable:
        return self.checks.tables[self.layer.device]


@dataclass
class _Pending:
    state: torch.Tensor              # pinned host copies
    capture: Dict[str, torch.Tensor]
    done: Optional[torch.cuda.Event]
    window: Optional[list]


class StepChecks:
    """Base of the per-step serving checks.  Subclasses set DETECTOR, COLS and CAPTURE (name -> dtype; widths come
    from the layers, via _register(widths=...)), READ_CAPTURE (the capture tensors read back with every poll, small
    ones; the others are read on demand), and implement _judge(layer, keys, captured, window) -> events and
    _count(layer, keys) (statistics)."""

    DETECTOR = ""
    COLS = 0
    CAPTURE: Dict[str, torch.dtype] = {}
    READ_CAPTURE: Tuple[str, ...] = ()
    FIRST_ROWS = 16                  # table rows allocated on a device's first layer

    def __init__(self, guard=None):
        self.guard = guard
        self.layers: List[Registered] = []
        self.unsupported: Dict[str, str] = {}
        self.tables: Dict[torch.device, DeviceTable] = {}
        self.events: list = []
        self.stats: dict = {"layers": 0, "alerts": 0}
        self.marked: Optional[int] = None          # the last step marked (None: steps are not marked)
        self._first_unread: Dict[torch.device, int] = {}
        self._last_clean: Dict[str, list] = {}
        self._pending: Dict[torch.device, _Pending] = {}
        self._lock = threading.RLock()

    # --------------------------------------------------------------------------------------------- registering
    def _register(self, name: str, module, device, widths: Optional[Dict[str, int]] = None, **info) -> Binding:
        device = torch.device(device)
        with self._lock:
            tab = self.tables.get(device)
            slot = sum(1 for lay in self.layers if lay.device == device)
            widths = dict(widths or {})
            if tab is None:
                tab = self.tables[device] = DeviceTable(
                    device, self.COLS, self.FIRST_ROWS, {k: (dt, widths.get(k, 1)) for k, dt in self.CAPTURE.items()})
            tab.fit(slot + 1, widths)
            self.layers.append(Registered(name, module, device, slot, dict(info)))
            self.stats["layers"] += 1
            return Binding(self, len(self.layers) - 1)

    def _refuse(self, name: str, why: str) -> None:
        self.unsupported[name] = why

    def table_row(self, b: Binding) -> int:
        return b.layer.slot

    # ----------------------------------------------------------------------------------------------- the steps
    def mark_step(self, step: int, rows: Optional[int] = None) -> None:
        """Before a model step: its number and, when known, its real rows (before padding to a graph's batch)."""
        self.marked = int(step) & M32
        for dev, tab in self.tables.items():
            tab.word.write(self.marked, rows, True)
            self._first_unread.setdefault(dev, self.marked)

    def end_step(self) -> None:
        """After a model step: calls until the next mark (warm-up, graph capture) are not the model's steps."""
        if self.marked is None:
            return
        for tab in self.tables.values():
            tab.word.write(self.marked, None, False)

    def _window(self, dev) -> Optional[list]:
        """The steps the rows read now cover: from the first step marked since the last read to the last marked."""
        if self.marked is None:
            return None
        first = self._first_unread.pop(dev, None)
        return [self.marked if first is None else first, self.marked]

    # --------------------------------------------------------------------------------------------- reading back
    def _snapshot(self, dev, tab: DeviceTable, wait: bool) -> _Pending:
        names = [k for k in self.READ_CAPTURE if k in tab.capture]
        if wait or not tab.state.is_cuda:
            p = _Pending(tab.state.to("cpu", copy=True), {k: tab.capture[k].to("cpu", copy=True) for k in names},
                         None, self._window(dev))
        else:
            st = torch.empty(tab.state.shape, dtype=tab.state.dtype, pin_memory=True)
            st.copy_(tab.state, non_blocking=True)
            caps = {}
            for k in names:
                caps[k] = torch.empty(tab.capture[k].shape, dtype=tab.capture[k].dtype, pin_memory=True)
                caps[k].copy_(tab.capture[k], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(dev))
            p = _Pending(st, caps, ev, self._window(dev))
        tab.state.zero_()                          # in stream order: calls queued later count in the next read
        return p

    def poll(self, wait: bool = False) -> list:
        """Alerts of the rows read back.  Without wait, the copy started now is reported by a later poll (none is
        waited for); with wait, everything queued so far is reported."""
        out = []
        with self._lock:
            for dev, tab in list(self.tables.items()):
                p = self._pending.get(dev)
                if p is not None and (wait or p.done is None or p.done.query()):
                    if p.done is not None:
                        p.done.synchronize()
                    del self._pending[dev]
                    out += self._report(dev, p)
                    p = None
                if wait:
                    out += self._report(dev, self._snapshot(dev, tab, True))
                elif p is None:
                    self._pending[dev] = self._snapshot(dev, tab, False)
        return out

    def _report(self, dev, p: _Pending) -> list:
        out = []
        for lay in self.layers:
            if lay.device != dev or lay.slot >= p.state.shape[0]:
                continue
            keys = [int(v) for v in p.state[lay.slot].tolist()]
            self._count(lay, keys)
            cap = {k: v[lay.slot] for k, v in p.capture.items()}
            evs = self._judge(lay, keys, cap, p.window)
            if not evs and p.window is not None and self._judged(keys):
                self._last_clean[lay.name] = list(p.window)
            out += evs
        return out

    def last_clean(self, name: str) -> Optional[list]:
        return self._last_clean.get(name)

    # ----------------------------------------------------------------------------------------------- the rest
    def detach(self) -> None:
        """Read what is left, then forget every layer."""
        try:
            if self.tables:
                self.poll(wait=True)
        finally:
            for lay in self.layers:
                self._unbind(lay)
            self.layers.clear()
            self.tables.clear()
            self._pending.clear()
            self._first_unread.clear()

    def coverage(self) -> dict:
        return {"layers": len(self.layers),
                "layers_checked": sum(1 for lay in self.layers if lay.calls > 0),
                "never_checked": sorted(lay.name for lay in self.layers if lay.calls == 0),
                "not_attached": dict(self.unsupported)}

    def emit(self, lay: Registered, z: float, row: Optional[int], detail: dict) -> object:
        from .serve import SDCEvent
        ev = SDCEvent(detector=self.DETECTOR, layer=lay.name, z=z, row=row, extra=detail)
        self.stats["alerts"] += 1
        self.events.append(ev)
        cb = getattr(self.guard, "on_alert", None)
        if cb:
            try:
                cb(ev)
            except Exception:  # noqa: BLE001  (an alert callback never breaks serving)
                pass
        return ev

    # ------------------------------------------------------------------------------------------ subclass hooks
    def _count(self, lay: Registered, keys: list) -> None:
        raise NotImplementedError

    def _judged(self, keys: list) -> bool:
        """Whether a clean row read back judged anything (for the last clean window)."""
        return True

    def _judge(self, lay: Registered, keys: list, captured: dict, window: Optional[list]) -> list:
        raise NotImplementedError

    def _unbind(self, lay: Registered) -> None:
        pass
