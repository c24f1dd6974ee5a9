"""Weight fingerprints (reference: serve_weights.py:73-86, :151-216).

fingerprint(t) -> int64[2] on t's device: the sum of t's raw bit values x_i and the sum of x_i * k(i), mod 2^64,
with k(i) = fmix64(i ^ 0x2545F4914F6CDD1D) (MurmurHash3's finalizer); values are int16 for 2-byte dtypes, int32 for
4-byte (and the two halves of 8-byte) ones, uint8 for 1-byte ones.  One HIP kernel pass (sdc_fingerprint2).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

KEY_SEED = 0x2545F4914F6CDD1D
MIX1 = 0xFF51AFD7ED558CCD
MIX2 = 0xC4CEB9FE1A85EC53


def _int_view(t: torch.Tensor):
    """(flat integer view, kind) of a tensor's raw bits (serve_weights.py:151-161); kind as sdc_fingerprint2."""
    flat = t.detach().contiguous().view(-1)
    es = flat.element_size()
    if es == 2:
        return flat.view(torch.int16), 0
    if es == 4:
        return flat.view(torch.int32), 1
    if es == 8:
        return flat.view(torch.int64).view(torch.int32), 1
    return flat.view(torch.uint8), 2


def fingerprint(t: Optional[torch.Tensor], out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[2] int64 (serve_weights.py:172-185).  A missing or empty tensor gives zeros on the CPU."""
    if not isinstance(t, torch.Tensor) or t.numel() == 0:
        return torch.zeros(2, dtype=torch.int64)
    _lib.require_gpu(t)
    v, kind = _int_view(t)
    if out is None:
        out = torch.zeros(2, dtype=torch.int64, device=v.device)
    rc = _lib.lib().sdc_fingerprint2(v.data_ptr(), v.numel(), kind, out.data_ptr(), _lib.stream_of(v))
    _lib.check(rc, "sdc_fingerprint2")
    return out


# ---------------------------------------------------------------------------------------------------------------
# The scheduled weight scan (serve_weights.py:389-972) and the model digest (:335-364)
#
# Each read of the guard's results fingerprints the next registered layers' tensors, up to a byte budget, on the
# GPU and compares them with their reference fingerprints: every registered tensor is compared once per pass over
# the model, so a changed bit that persists until its layer's turn is named however small its effect on outputs.
# References are provisional until their first comparison (a reload that processed weights in temporary tensors
# and copied them into the originals is taken in again); after it, tensors that moved, or that share memory with
# another entry's (CPU offloading), are left out rather than called changed.  A read's comparisons come back
# through pinned host memory and an event, so no read waits for the GPU (unless asked to).  Repair keeps a host copy
# of each entry and writes it back in place when at most REPAIR_MAX_VALUES values differ, then verifies it.

import hashlib
import json
import logging
import time
from dataclasses import dataclass, field
from typing import Callable, Sequence

log = logging.getLogger("sdcguard")

CHUNK = 1 << 20                         # values compared per host step of a repair's count
DEFAULT_BUDGET_MB = 64.0
DEFAULT_MAX_MB = 1024.0                 # the most a read compares to meet a verification-age target
REPAIR_MAX_VALUES = 64                  # a fault changes a few values; an unannounced update changes most of them
HOST_SHARE = 0.5                        # host copies take at most this share of free host memory per local GPU


def _host_room() -> Optional[int]:
    """Bytes of host memory free for this process: MemAvailable, or the cgroup's limit less its use when lower;
    None when neither can be read."""
    room = None
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    room = int(line.split()[1]) * 1024
                    break
    except (OSError, ValueError, IndexError):
        pass
    for lim_path, use_path in (("/sys/fs/cgroup/memory.max", "/sys/fs/cgroup/memory.current"),
                               ("/sys/fs/cgroup/memory/memory.limit_in_bytes",
                                "/sys/fs/cgroup/memory/memory.usage_in_bytes")):
        try:
            with open(lim_path) as f:
                lim = f.read().strip()
            if lim == "max":
                continue
            with open(use_path) as f:
                left = int(lim) - int(f.read().strip())
            room = left if room is None else min(room, left)
            break
        except (OSError, ValueError):
            continue
    return room


def _local_gpus() -> int:
    import os
    try:
        n = int(os.environ.get("LOCAL_WORLD_SIZE") or 0)
    except ValueError:
        n = 0
    if n <= 0:
        n = torch.cuda.device_count() if torch.cuda.is_available() else 1
    return max(1, n)


def _location(t) -> Optional[tuple]:
    if not isinstance(t, torch.Tensor) or t.numel() == 0:
        return None
    return str(t.device), t.data_ptr(), tuple(t.shape), t.dtype


def _bias(m) -> Optional[torch.Tensor]:
    b = getattr(m, "bias", None)
    return b if isinstance(b, torch.Tensor) else None


def fingerprints(tensors: Sequence[Optional[torch.Tensor]], device) -> torch.Tensor:
    """[k, 2] int64 on `device`: each tensor's fingerprint (a missing or empty tensor's row is zeros), one library
    launch per tensor into its row; no host synchronisation."""
    device = torch.device(device)
    out = torch.zeros(len(tensors), 2, dtype=torch.int64, device=device)
    for i, t in enumerate(tensors):
        if not (isinstance(t, torch.Tensor) and t.numel()):
            continue
        if t.device == device:
            fingerprint(t, out=out[i])
        else:
            out[i] = fingerprint(t).to(device)
    return out


def param_tensors(name: str, p):
    """A parameter's tensors as digests take them: a shared-weight parameter's partitions, a tensor subclass's inner
    tensors, else the parameter itself (serve_weights.py:315-332)."""
    parts = getattr(p, "partitions", None)
    if isinstance(parts, dict) and parts:
        for k, v in parts.items():
            yield from param_tensors(f"{name}.{k}", v)
        return
    try:
        from torch.utils._python_dispatch import is_traceable_wrapper_subclass
        wrapped = is_traceable_wrapper_subclass(p)
    except Exception:  # noqa: BLE001
        wrapped = False
    if wrapped:
        for a in p.__tensor_flatten__()[0]:
            yield from param_tensors(f"{name}.{a}", getattr(p, a))
        return
    yield name, p


def model_digest(model) -> Optional[str]:
    """One identity of a loaded model's weights (serve_weights.py:335-364): every parameter tensor (once)
    fingerprinted, then names, shapes, dtypes and fingerprints hashed in name order (SHA-256, 16 hex digits; the
    same text as the reference's, so the two give the same digest).  None without parameters."""
    named, seen = [], set()
    for pname, p in model.named_parameters():
        for tname, t in param_tensors(pname, p):
            if isinstance(t, torch.Tensor) and id(t) not in seen:
                seen.add(id(t))
                named.append((tname, t))
    if not named:
        return None
    named.sort(key=lambda x: x[0])
    rows: list = [None] * len(named)
    by_dev: dict = {}
    for i, (_, t) in enumerate(named):
        by_dev.setdefault(t.device, []).append(i)
    with torch.no_grad():
        for dev, idx in by_dev.items():
            got = fingerprints([named[i][1] for i in idx], dev).cpu().tolist()
            for i, f in zip(idx, got):
                rows[i] = f
    h = hashlib.sha256()
    for (n, t), f in zip(named, rows):
        h.update(json.dumps([n, list(t.shape), str(t.dtype).replace("torch.", ""), f]).encode())
    return h.hexdigest()[:16]


def before_repair(restored: Optional[dict], step) -> bool:
    """Whether an output of `step` (None: unknown) may predate a weight repair recorded as `restored`."""
    if restored is None:
        return False
    at = restored.get("step")
    return step is None or at is None or step <= at


def repair_why(restored: dict, step) -> str:
    return (f"the weight repair wrote this layer's load-time weights back after step {restored.get('step')}, and "
            f"this output (step {step}) may have been computed before that, with the changed weights: a recheck with "
            "the weights as they are now can't say whether it was right")


@dataclass
class _Entry:
    """One registered group of tensors (a layer's weight and bias, or a quantized layer's tensors)."""
    name: str
    get: Callable
    kind: str
    module: object
    device: torch.device
    nbytes: int
    ref: Optional[torch.Tensor] = None        # [k, 2] int64 on the device
    at: list = field(default_factory=list)    # where the tensors were when the reference was taken
    ids: list = field(default_factory=list)
    provisional: bool = True
    ref_step: Optional[int] = None
    gen: int = -1                             # bumped with every new reference: older comparisons are void
    alerted: bool = False
    excluded: Optional[str] = None
    last_clean: Optional[float] = None
    last_clean_step: Optional[int] = None
    compared: int = 0
    since: float = field(default_factory=time.monotonic)
    repairs: int = 0
    compared_at_repair: int = -1
    clean: Optional[list] = None              # repair: host copies of the tensors the reference fingerprints


@dataclass
class _Batch:
    """One read's comparisons on one device, on their way to the host."""
    flags: torch.Tensor                       # pinned int32 per entry (or on the host already)
    event: Optional[object]
    items: list                               # (entry index, step, generation)


class WeightScan:
    """Scheduled weight integrity of one serving guard (ServeGuard.weight_scan()); poll() runs at each of the
    guard's reads (serve_weights.py:389-972)."""

    def __init__(self, guard=None, budget_mb: float = DEFAULT_BUDGET_MB, target_age: Optional[float] = None,
                 max_mb: float = DEFAULT_MAX_MB, max_gap: float = 4.0, repair: bool = False,
                 repair_max_values: int = REPAIR_MAX_VALUES, host_allowance: Optional[int] = None):
        self.guard = guard
        self.repair = bool(repair)
        self.repair_max_values = max(0, int(repair_max_values))
        self.repair_off: Optional[str] = None
        self._host_allowance = host_allowance
        self._to_repair: list = []            # (entry index, generation, alert window, last clean)
        self.budget = max(1, int(float(budget_mb) * (1 << 20)))
        self.target_age = float(target_age) if target_age else None
        self.max_budget = max(self.budget, int(float(max_mb) * (1 << 20)))
        self.max_gap = float(max_gap)
        self._last_read: Optional[float] = None
        self._interval: Optional[float] = None
        self._age_warned = False
        self.entries: list = []
        self._slots: set = set()
        self.cursor = 0
        self.paused = False
        self._pending: dict = {}              # device -> [_Batch]
        self._pass_started = time.monotonic()
        self.not_scanned: dict = {}
        self.events: list = []
        self.stats = {"entries": 0, "bytes": 0, "reads": 0, "entries_compared": 0, "bytes_compared": 0,
                      "passes": 0, "last_pass_seconds": None, "changed": 0, "alerts": 0, "references_retaken": 0,
                      "budget_bytes_now": self.budget, "target_met": None, "repaired": 0, "repair_failed": 0,
                      "host_copy_bytes": 0}

    # ------------------------------------------------------------------------------------------- entries
    def add(self, name: str, get: Callable[[], Sequence[Optional[torch.Tensor]]], kind: str,
            module: Optional[torch.nn.Module] = None) -> Optional[int]:
        """Register tensors (get() returns them as they are now); their fingerprint now is the provisional
        reference.  kind: "checked", "quantized", "unchecked" or "other".  The entry's index, or None."""
        tensors = list(get())
        live = [t for t in tensors if isinstance(t, torch.Tensor) and t.numel()]
        if not live:
            self.not_scanned[name] = "no weight tensors to compare"
            return None
        e = _Entry(name=name, get=get, kind=kind, module=module, device=live[0].device,
                   nbytes=sum(t.numel() * t.element_size() for t in live))
        with torch.inference_mode(False), torch.no_grad():
            self._take_reference(e, tensors)
        self.entries.append(e)
        self.stats["entries"] = len(self.entries)
        self.stats["bytes"] += e.nbytes
        self.not_scanned.pop(name, None)
        return len(self.entries) - 1

    def sync(self) -> None:
        """Take in the guard's checked layers registered since the last call."""
        g = self.guard
        layers = getattr(g, "layers", None) or []
        for slot, lay in enumerate(layers):
            if slot in self._slots:
                continue
            self._slots.add(slot)
            mod = lay["module"]
            self.add(lay["name"], (lambda m=mod: (getattr(m, "weight", None), _bias(m))), "checked", mod)

    def refresh(self, module: Optional[torch.nn.Module] = None, kind: Optional[str] = None,
                name: Optional[str] = None) -> int:
        """After an intended update: the selected entries (all by default) take new provisional references and are
        compared again.  Comparisons started before, and repairs not yet made, are dropped."""
        n = 0
        self._pending.clear()
        now = time.monotonic()
        with torch.inference_mode(False), torch.no_grad():
            for e in self.entries:
                if (module is not None and e.module is not module) or (kind is not None and e.kind != kind) or \
                        (name is not None and e.name != name):
                    continue
                self._take_reference(e, list(e.get()))
                e.alerted, e.excluded, e.last_clean, e.last_clean_step, e.since = False, None, None, None, now
                self.not_scanned.pop(e.name, None)
                n += 1
        self._to_repair = [r for r in self._to_repair if r[1] == self.entries[r[0]].gen]
        return n

    def _take_reference(self, e: _Entry, tensors: list) -> None:
        e.ref = fingerprints(tensors, e.device)
        e.at = [_location(t) for t in tensors]
        e.ids = [id(t) for t in tensors]
        e.provisional = True
        e.ref_step = getattr(self.guard, "_marked_step", None)
        e.gen += 1
        if self.repair:
            self._keep_copy(e, tensors)

    @staticmethod
    def _nbytes(ts) -> int:
        return sum(c.numel() * c.element_size() for c in ts or () if c is not None)

    def _keep_copy(self, e: _Entry, tensors: list) -> None:
        """e.clean: host copies of the tensors (an existing copy of the same shape and dtype is overwritten).
        Repair turns itself off for every entry when the copies would pass the host allowance."""
        old = e.clean or []
        same = [k < len(old) and old[k] is not None and isinstance(t, torch.Tensor) and t.numel() > 0 and
                old[k].shape == t.shape and old[k].dtype == t.dtype for k, t in enumerate(tensors)]
        need = sum(t.numel() * t.element_size() for t, s in zip(tensors, same)
                   if isinstance(t, torch.Tensor) and t.numel() and not s)
        freed = self._nbytes(c for k, c in enumerate(old) if not (k < len(same) and same[k]))
        if self._host_allowance is None:
            room = _host_room()
            if room is None:
                self._host_allowance = 0
                self._repair_disable("the free host memory can't be read, so the host copies can't be sized safely")
                return
            self._host_allowance = int(HOST_SHARE * max(room, 0) / _local_gpus())
        after = self.stats["host_copy_bytes"] - freed + need
        if after > self._host_allowance:
            self._repair_disable(f"the host copies would take {after / (1 << 30):.2f} GiB, more than this worker's "
                                 f"allowance of {self._host_allowance / (1 << 30):.2f} GiB")
            return
        clean = []
        for k, (t, s) in enumerate(zip(tensors, same)):
            if not (isinstance(t, torch.Tensor) and t.numel()):
                clean.append(None)
            elif s:
                old[k].copy_(t.detach())
                clean.append(old[k])
            else:
                clean.append(t.detach().to("cpu", copy=True))
        e.clean = clean
        self.stats["host_copy_bytes"] = after

    def _repair_disable(self, why: str) -> None:
        self.repair, self.repair_off = False, why
        for e in self.entries:
            e.clean = None
        self.stats["host_copy_bytes"] = 0
        self._to_repair = []
        log.warning("sdcguard: weight repair is off: %s; the scan still compares and alerts", why)

    def _drop_copy(self, e: _Entry) -> None:
        if e.clean:
            self.stats["host_copy_bytes"] -= self._nbytes(e.clean)
            e.clean = None

    def _shared(self, e: _Entry, tensors: list) -> tuple:
        """(why, the other entry) when another entry's different tensor lives at the same address."""
        mine = {}
        for t in tensors:
            loc = _location(t)
            if loc:
                mine[(loc[0], loc[1])] = id(t)
        for other in self.entries:
            if other is e:
                continue
            for loc, oid in zip(other.at, other.ids):
                if loc and mine.get((loc[0], loc[1]), oid) != oid:
                    return f"shares its memory with {other.name}'s tensors (CPU offloading)", other
        return None, None

    def _exclude(self, e: _Entry, why: str) -> None:
        if e.excluded is None:
            log.warning("sdcguard: the weight scan no longer compares %s: %s", e.name, why)
        e.excluded = why
        self.not_scanned[e.name] = why
        self._drop_copy(e)

    # ------------------------------------------------------------------------------------------- reads
    def poll(self, wait: bool = False) -> list:
        """Report the comparisons that have come back and start the next ones (up to the byte budget)."""
        self.sync()
        self.stats["reads"] += 1
        now = time.monotonic()
        if self._last_read is not None:
            dt = min(now - self._last_read, self.max_gap)
            self._interval = dt if self._interval is None else 0.8 * self._interval + 0.2 * dt
        self._last_read = now
        events = self._collect(wait)
        if self.entries and not self.paused:
            events += self._start(wait)
        if self._to_repair:
            self._repair_pending()
        return events

    def target(self) -> int:
        """The bytes this read compares: the budget, or with a verification-age target enough that a pass over the
        entries still compared takes at most 2/3 of it at the measured time between reads, up to max_mb."""
        if not self.target_age or self._interval is None or self._interval <= 0:
            return self.budget
        live = sum(e.nbytes for e in self.entries if not e.alerted and not e.excluded)
        reads = max(1.0, (self.target_age * 2 / 3) / self._interval)
        want = int(live / reads) + 1
        met = want <= self.max_budget
        if not met and not self._age_warned:
            self._age_warned = True
            log.warning("sdcguard: the weight scan can't compare every weight within %gs at %.2fs between reads "
                        "(it would need %.0f MB a read, above the %.0f MB most)", self.target_age, self._interval,
                        want / (1 << 20), self.max_budget / (1 << 20))
        self.stats["target_met"] = met
        return max(self.budget, min(want, self.max_budget))

    def oldest_age(self, now: Optional[float] = None) -> Optional[float]:
        now = time.monotonic() if now is None else now
        ages = [now - (e.last_clean if e.last_clean is not None else e.since)
                for e in self.entries if not e.alerted and not e.excluded]
        return max(ages) if ages else None

    def _start(self, wait: bool) -> list:
        """Fingerprint the next entries (round robin, up to the budget) and queue their comparison: per device one
        stacked comparison with the references and one per-entry reduction."""
        chosen: dict = {}                      # device -> [(entry index, step, gen, tensors)]
        spent, tried, n = 0, 0, len(self.entries)
        budget = self.target()
        self.stats["budget_bytes_now"] = budget
        step = getattr(self.guard, "_marked_step", None)
        with torch.inference_mode(False), torch.no_grad():
            while tried < n and (spent < budget or not chosen):
                i = self.cursor
                self.cursor = (self.cursor + 1) % n
                tried += 1
                if self.cursor == 0:
                    self._pass_done()
                e = self.entries[i]
                if e.alerted or e.excluded:
                    continue
                tensors = list(e.get())
                why, other = self._shared(e, tensors)
                if why:
                    self._exclude(e, why)
                    if other is not None and not other.excluded:
                        self._exclude(other, f"shares its memory with {e.name}'s tensors (CPU offloading)")
                    continue
                if [_location(t) for t in tensors] != e.at:
                    if e.provisional:            # never compared: take the reference again where they are now
                        self._take_reference(e, tensors)
                        self.stats["references_retaken"] += 1
                        continue
                    self._exclude(e, "its tensors moved or changed shape after they were compared (call refresh() "
                                     "after an intended reload)")
                    continue
                chosen.setdefault(e.device, []).append((i, step, e.gen, tensors))
                spent += e.nbytes
            events = []
            for dev, items in chosen.items():
                tensors = [t for *_, ts in items for t in ts]
                owner = torch.tensor([k for k, it in enumerate(items) for _ in it[3]], dtype=torch.int64)
                owner = owner.pin_memory().to(dev, non_blocking=True) if dev.type == "cuda" else owner
                now = fingerprints(tensors, dev)
                refs = torch.cat([self.entries[i].ref for i, *_ in items])
                differ = torch.ne(now, refs).any(-1).to(torch.int32)
                flags = torch.zeros(len(items), dtype=torch.int32, device=dev).index_add_(0, owner, differ)
                idx = [(i, s, g) for i, s, g, _ in items]
                if dev.type == "cuda" and not wait:
                    host = torch.empty(flags.shape, dtype=torch.int32, pin_memory=True)
                    host.copy_(flags, non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(torch.cuda.current_stream(dev))
                    self._pending.setdefault(dev, []).append(_Batch(host, ev, idx))
                else:
                    events += self._judge(flags.cpu(), idx)
                self.stats["entries_compared"] += len(idx)
                self.stats["bytes_compared"] += sum(self.entries[i].nbytes for i, _, _ in idx)
        return events

    def _pass_done(self) -> None:
        now = time.monotonic()
        self.stats["passes"] += 1
        self.stats["last_pass_seconds"] = round(now - self._pass_started, 3)
        self._pass_started = now

    def _collect(self, wait: bool) -> list:
        events = []
        for dev in list(self._pending):
            left = []
            for b in self._pending[dev]:
                if wait:
                    b.event.synchronize()
                if b.event.query():
                    events += self._judge(b.flags, b.items)
                else:
                    left.append(b)
            if left:
                self._pending[dev] = left
            else:
                del self._pending[dev]
        return events

    def _judge(self, flags: torch.Tensor, items: list) -> list:
        events = []
        now = time.monotonic()
        for f, (i, step, gen) in zip(flags.tolist(), items):
            e = self.entries[i]
            if e.excluded or gen != e.gen:      # left out, or a new reference, since this comparison started
                continue
            e.compared += 1
            e.provisional = False
            if not f:
                e.last_clean, e.last_clean_step = now, step
                continue
            if e.alerted:
                continue
            e.alerted = True
            self.stats["changed"] += 1
            ev = self._alert(e, now, step)
            events.append(ev)
            if self.repair and e.clean:
                self._to_repair.append((i, e.gen, ev.extra.get("read_window_steps"),
                                        ev.extra.get("last_clean_read_steps")))
        return events

    # ------------------------------------------------------------------------------------------- repair
    def _repair_pending(self) -> None:
        """Entries found changed with repair on: when at most repair_max_values values differ from the host copy, it
        is written back in place (after the work queued so far) and verified against the reference at once; a
        record goes out either way (the alert that found the change stands)."""
        todo, self._to_repair = self._to_repair, []
        for i, gen, window, clean in todo:
            e = self.entries[i]
            if gen != e.gen or not e.alerted:
                continue
            at = getattr(self.guard, "_marked_step", None)
            counts = None
            try:
                with torch.inference_mode(False), torch.no_grad():
                    ok, why, counts = self._restore(e, at)
            except Exception as ex:  # noqa: BLE001  (a failed repair leaves the alert as it was)
                ok, why = False, f"the restore failed: {type(ex).__name__}: {ex}"[:300]
            if ok:
                e.alerted = False
                e.repairs += 1
                e.gen += 1
                e.last_clean, e.last_clean_step = time.monotonic(), at
                e.compared_at_repair = e.compared
                self.stats["repaired"] += 1
            else:
                self.stats["repair_failed"] += 1
            self._emit(self._repair_event(e, ok, why, at, window, clean, counts))

    def _count_changed(self, pairs: list) -> tuple:
        """(values that differ from the copy, stopped early), CHUNK values at a time on the host."""
        changed = 0
        for t, c in pairs:
            tv = t.detach().contiguous().view(-1).view(torch.uint8)
            cv = c.contiguous().view(-1).view(torch.uint8)
            es = max(1, min(t.element_size(), 4))
            tv = tv.view({1: torch.uint8, 2: torch.int16, 4: torch.int32}[es])
            cv = cv.view({1: torch.uint8, 2: torch.int16, 4: torch.int32}[es])
            for a in range(0, tv.numel(), CHUNK):
                changed += int(torch.ne(tv[a:a + CHUNK].to("cpu"), cv[a:a + CHUNK]).sum())
                if changed > self.repair_max_values:
                    return changed, True
        return changed, False

    def _restore(self, e: _Entry, at=None) -> tuple:
        if e.excluded:
            return False, f"the scan no longer compares it: {e.excluded}", None
        tensors = list(e.get())
        clean = e.clean or []
        if [_location(t) for t in tensors] != e.at or len(clean) != len(tensors):
            return False, "its tensors moved or changed since the clean copy was taken", None
        why, _ = self._shared(e, tensors)
        if why:
            return False, f"it {why}", None
        pairs = []
        for t, c in zip(tensors, clean):
            if c is None or not isinstance(t, torch.Tensor):
                continue
            if t.shape != c.shape or t.dtype != c.dtype:
                return False, "a tensor's shape or dtype differs from its clean copy", None
            pairs.append((t, c))
        if e.device.type == "cuda":
            torch.cuda.synchronize(e.device)
        changed, stopped = self._count_changed(pairs)
        values = sum(c.numel() * (2 if c.element_size() == 8 else 1) for _, c in pairs)   # (8 bytes: two words)
        counts = {"values_changed": changed, "values": values, "at_least": stopped}
        if changed > self.repair_max_values:
            return False, (f"{'at least ' if stopped else ''}{changed} values differ from the copy kept with the "
                           f"reference, more than a fault in memory would change (repair writes back at most "
                           f"{self.repair_max_values}): an update the guard wasn't told about, or a stray write"), counts
        try:
            for t, c in pairs:
                if t.is_inference():
                    with torch.inference_mode():
                        t.copy_(c)
                else:
                    with torch.inference_mode(False), torch.no_grad():
                        t.copy_(c)
        finally:
            restored = getattr(self.guard, "_weights_restored", None)
            if restored is not None and e.module is not None:
                try:
                    restored(e.module, at)
                except Exception:  # noqa: BLE001
                    pass
        if e.device.type == "cuda":
            torch.cuda.synchronize(e.device)
        now = fingerprints(tensors, e.device)
        if torch.equal(now.cpu(), e.ref.cpu()):
            return True, None, counts
        return False, "the restored weights still don't match their reference fingerprint", counts

    # ------------------------------------------------------------------------------------------- reports
    def _emit(self, ev) -> None:
        self.events.append(ev)
        g = self.guard
        if g is not None and getattr(g, "events", None) is not None and g.events is not self.events:
            g.events.append(ev)
        cb = getattr(g, "on_alert", None) if g is not None else None
        if cb:
            try:
                cb(ev)
            except Exception:  # noqa: BLE001  (an alert callback never breaks serving)
                pass

    def _alert(self, e: _Entry, now: float, step: Optional[int]):
        from .serve import SDCEvent
        clean = e.last_clean_step
        window, since = None, None
        if step is not None:
            if clean is not None:
                start, since = (clean + 1 if clean < step else step), "the last clean comparison"
            else:
                start = min(e.ref_step + 1, step) if e.ref_step is not None else 0
                since = "the reference (at load or the last refresh)" if e.ref_step is not None else "load"
            window = [start, step]
        detail = {"where": e.name, "finding": "weights_changed", "kind": e.kind, "weights_changed_since_load": True,
                  "recheck": {"verdict": "weights_changed",
                              "why": "the layer's tensors no longer match their reference fingerprint (taken at "
                                     "load, or at the last refresh)"},
                  "read_window_steps": window, "window_since": since,
                  "last_clean_read_steps": [clean, clean] if clean is not None else None,
                  "seconds_since_last_clean_comparison": (round(now - e.last_clean, 3)
                                                          if e.last_clean is not None else None),
                  "last_pass_seconds": self.stats["last_pass_seconds"],
                  "scan": {"budget_bytes": self.stats["budget_bytes_now"], "entries": len(self.entries),
                           "target_age_seconds": self.target_age},
                  "reading": "a weight bit changed after load: memory corruption, or an update the guard wasn't "
                             "told about (call refresh() after an intended one). Every request this layer served "
                             "since its last clean comparison may have used the changed weights."}
        ev = SDCEvent(detector="serve_weights", layer=e.name, z=float("inf"), extra=detail)
        self.stats["alerts"] += 1
        self._emit(ev)
        return ev

    def _repair_event(self, e: _Entry, ok: bool, why, at, window, clean, counts):
        from .serve import SDCEvent
        n = (counts or {}).get("values_changed")
        start = window[0] if window else at
        detail = {"where": e.name, "kind": e.kind, "finding": "weights_restored" if ok else "weights_restore_failed",
                  "recheck": {"verdict": "weights_restored" if ok else "restore_failed",
                              "why": "the copy kept with the reference was written back and the tensors match their "
                                     "reference fingerprint again" if ok else why},
                  "repairs": e.repairs, "values_changed": n, "values": (counts or {}).get("values"),
                  "values_changed_at_least": bool((counts or {}).get("at_least")), "repaired_at_step": at,
                  "read_window_steps": [start, at] if start is not None and at is not None and start <= at else None,
                  "last_clean_read_steps": clean,
                  "reading": ("restored in place and verified; requests this layer served from its last clean "
                              "comparison to the repair may have used the changed weights" if ok else
                              f"not restored ({why}): the layer keeps its changed weights")}
        (log.warning if ok else log.error)("sdcguard: weight repair of %s: %s", e.name,
                                           f"restored ({n} values) and verified" if ok else why)
        return SDCEvent(detector="serve_weights", layer=e.name, z=0.0 if ok else float("inf"), extra=detail)

    def coverage(self) -> dict:
        by_kind: dict = {}
        for e in self.entries:
            by_kind[e.kind] = by_kind.get(e.kind, 0) + 1
        age = self.oldest_age()
        return {"entries": len(self.entries), "by_kind": by_kind, "bytes": self.stats["bytes"],
                "budget_bytes_per_read": self.budget, "budget_bytes_now": self.stats["budget_bytes_now"],
                "target_age_seconds": self.target_age, "target_met": self.stats["target_met"],
                "oldest_verification_age_seconds": round(age, 3) if age is not None else None,
                "oldest_within_target": (age <= self.target_age) if self.target_age and age is not None else None,
                "passes": self.stats["passes"], "last_pass_seconds": self.stats["last_pass_seconds"],
                "never_compared": sorted(e.name for e in self.entries if not e.compared and not e.excluded),
                "repair": {"on": self.repair, "off_because": self.repair_off, "max_values": self.repair_max_values,
                           "host_copy_bytes": self.stats["host_copy_bytes"],
                           "host_allowance_bytes": self._host_allowance, "repaired": self.stats["repaired"],
                           "failed": self.stats["repair_failed"],
                           "entries_repaired": sorted(e.name for e in self.entries if e.repairs),
                           "not_compared_since_repair": sorted(e.name for e in self.entries if e.repairs and
                                                               not e.excluded and e.compared <= e.compared_at_repair)},
                "changed": sorted(e.name for e in self.entries if e.alerted),
                "not_scanned": dict(self.not_scanned), "kernel": "sdc_fingerprint2"}
