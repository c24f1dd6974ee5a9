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
# The model digest (the reference's serve_weights.py:335-364 hashes the same text) and the scheduled weight scan
# (the reference's WeightScan, serve_weights.py:389-972, built here around a per-group status and a device-side
# comparison).
#
# The scan keeps, per registered group of tensors (a layer's weight and bias), a reference fingerprint on the GPU.
# Every read of the guard's results fingerprints the next groups in turn, up to a byte budget, and compares them
# with their references on the device; one int32 per group comes back through pinned memory and an event, so a read
# never waits for the GPU unless asked to.  Each group is compared once per pass over the model, so a bit that
# changes and stays changed is named within one pass, however small its effect on the outputs.
#
# A group's status moves PROVISIONAL (reference taken, never compared) -> CLEAN (compared equal) -> CHANGED (compared
# different: one alert) or EXCLUDED (its tensors moved, or share memory with another group's: never called changed).
# A provisional group whose tensors moved is taken in again where they are now (a load that processes weights in
# temporary tensors and copies them into place).  refresh() makes groups provisional again after an intended update.
# With repair on, a host copy of each group is kept; a changed group that differs from it in at most
# repair_max_values values is written back in place and verified against its reference.

import enum
import hashlib
import json
import logging
import os
import time
from dataclasses import dataclass, field
from typing import Callable, Iterator, List, Sequence, Tuple

log = logging.getLogger("sdcguard")

DEFAULT_BUDGET_MB = 64.0
DEFAULT_MAX_MB = 1024.0                 # the most one read compares to meet a verification-age target
REPAIR_MAX_VALUES = 64                  # a memory fault changes a few values; an update changes most of them
HOST_SHARE = 0.5                        # share of the free host memory (per local GPU) the repair copies may take
COUNT_CHUNK = 1 << 20                   # values compared per host step when a repair counts the changed values


def fingerprints(tensors: Sequence[Optional[torch.Tensor]], device) -> torch.Tensor:
    """[k, 2] int64 on `device`: row i the fingerprint of tensors[i] (zeros for a missing or empty one); one library
    launch per tensor, no host synchronisation."""
    device = torch.device(device)
    out = torch.zeros(len(tensors), 2, dtype=torch.int64, device=device)
    for i, t in enumerate(tensors):
        if isinstance(t, torch.Tensor) and t.numel():
            if t.device == device:
                fingerprint(t, out=out[i])
            else:
                out[i] = fingerprint(t).to(device)
    return out


def _leaves(name: str, p) -> Iterator[Tuple[str, torch.Tensor]]:
    """(name, tensor) of every tensor a parameter holds, depth first: a shared weight's partitions (name.key) and a
    tensor subclass's inner tensors (name.attr) stand for it; a plain tensor is itself."""
    todo = [(name, p)]
    while todo:
        n, t = todo.pop()
        parts = getattr(t, "partitions", None)
        if isinstance(parts, dict) and parts:
            todo.extend((f"{n}.{k}", v) for k, v in reversed(list(parts.items())))
            continue
        inner = None
        try:
            from torch.utils._python_dispatch import is_traceable_wrapper_subclass
            if is_traceable_wrapper_subclass(t):
                inner = t.__tensor_flatten__()[0]
        except Exception:  # noqa: BLE001  (not a subclass this torch can flatten: the tensor itself)
            inner = None
        if inner:
            todo.extend((f"{n}.{a}", getattr(t, a)) for a in reversed(list(inner)))
            continue
        yield n, t


param_tensors = _leaves


def model_digest(model) -> Optional[str]:
    """16 hex digits naming a loaded model's weights: SHA-256 over one JSON line per tensor, in name order,
    [name, shape, dtype, fingerprint] (every tensor once, however many parameters share it).  The text is the
    reference's (serve_weights.py:335-364), so both give a model the same digest.  None for a model without
    parameters."""
    tensors = {}
    for pname, p in model.named_parameters():
        for tname, t in _leaves(pname, p):
            if isinstance(t, torch.Tensor):
                tensors.setdefault(id(t), (tname, t))
    if not tensors:
        return None
    items = sorted(tensors.values(), key=lambda nt: nt[0])
    prints: dict = {}
    with torch.no_grad():
        for dev in {t.device for _, t in items}:
            mine = [(n, t) for n, t in items if t.device == dev]
            for (n, _), f in zip(mine, fingerprints([t for _, t in mine], dev).cpu().tolist()):
                prints[n] = f
    h = hashlib.sha256()
    for n, t in items:
        h.update(json.dumps([n, list(t.shape), str(t.dtype).replace("torch.", ""), prints[n]]).encode())
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


def _free_host_bytes() -> Optional[int]:
    """Host memory this process may still take: the available memory, or what the memory cgroup leaves when that is
    less; None when neither is known."""
    try:
        import psutil
        free = int(psutil.virtual_memory().available)
    except Exception:  # noqa: BLE001
        free = None
    for cap, used in (("/sys/fs/cgroup/memory.max", "/sys/fs/cgroup/memory.current"),
                      ("/sys/fs/cgroup/memory/memory.limit_in_bytes", "/sys/fs/cgroup/memory/memory.usage_in_bytes")):
        try:
            with open(cap) as f1, open(used) as f2:
                c, u = f1.read().strip(), f2.read().strip()
            if c != "max":
                left = int(c) - int(u)
                free = left if free is None else min(free, left)
                break
        except (OSError, ValueError):
            pass
    return free


def _gpus_on_host() -> int:
    """GPUs sharing this host's memory: LOCAL_WORLD_SIZE when a launcher set it, else the visible devices."""
    n = os.environ.get("LOCAL_WORLD_SIZE", "")
    if n.isdigit() and int(n) > 0:
        return int(n)
    return max(1, torch.cuda.device_count() if torch.cuda.is_available() else 1)


def _where(t) -> Optional[tuple]:
    """Where a tensor's values live (device, address, shape, dtype), or None for a missing or empty tensor."""
    if isinstance(t, torch.Tensor) and t.numel():
        return str(t.device), t.data_ptr(), tuple(t.shape), t.dtype
    return None


class Status(enum.Enum):
    PROVISIONAL = "provisional"     # reference taken, not yet compared
    CLEAN = "clean"                 # last comparison equal
    CHANGED = "changed"             # compared different (alerted once)
    EXCLUDED = "excluded"           # moved or shares memory: left out


@dataclass(eq=False)
class _Group:
    """One registered group of tensors: get() returns them as they are now."""
    name: str
    get: Callable
    kind: str
    module: object
    device: torch.device
    nbytes: int
    ref: Optional[torch.Tensor] = None         # [k, 2] int64 on the device
    places: list = field(default_factory=list)   # _where() of each tensor at the reference
    objects: list = field(default_factory=list)  # id() of each tensor at the reference
    gen: int = 0                               # bumped with every new reference: comparisons of an older one are void
    status: Status = Status.PROVISIONAL
    why_out: Optional[str] = None
    ref_step: Optional[int] = None
    clean_time: Optional[float] = None
    clean_step: Optional[int] = None
    since: float = field(default_factory=time.monotonic)
    compared: int = 0
    repairs: int = 0
    compared_at_repair: int = -1
    copies: Optional[list] = None              # repair: host copies of the tensors

    def tensors(self) -> list:
        return list(self.get())

    def live(self) -> bool:
        return self.status in (Status.PROVISIONAL, Status.CLEAN)


@dataclass
class _InFlight:
    flags: torch.Tensor                        # int32 per group: tensors whose fingerprint differs (pinned host)
    done: Optional[torch.cuda.Event]
    groups: list                               # (group, generation, step)


class _Copies:
    """The repair's host copies, within an allowance of host bytes."""

    def __init__(self, allowance: Optional[int]):
        self.allowance = allowance
        self.bytes = 0

    @staticmethod
    def size(copies) -> int:
        return sum(c.numel() * c.element_size() for c in copies or () if c is not None)

    def keep(self, g: _Group, tensors: list) -> Optional[str]:
        """Copy g's tensors to the host (reusing copies of the same shape and dtype); why repair must stop, or None."""
        if self.allowance is None:
            free = _free_host_bytes()
            if free is None:
                return "the free host memory can't be read, so the host copies can't be sized safely"
            self.allowance = int(HOST_SHARE * max(free, 0) / _gpus_on_host())
        old = g.copies or []
        reuse = [i < len(old) and old[i] is not None and isinstance(t, torch.Tensor) and t.numel() > 0 and
                 old[i].shape == t.shape and old[i].dtype == t.dtype for i, t in enumerate(tensors)]
        total = self.bytes - self.size(c for i, c in enumerate(old) if not (i < len(reuse) and reuse[i]))
        total += sum(t.numel() * t.element_size() for t, r in zip(tensors, reuse)
                     if isinstance(t, torch.Tensor) and t.numel() and not r)
        if total > self.allowance:
            return (f"the host copies would take {total / (1 << 30):.2f} GiB, more than this worker's allowance of "
                    f"{self.allowance / (1 << 30):.2f} GiB")
        copies = []
        for i, t in enumerate(tensors):
            if not (isinstance(t, torch.Tensor) and t.numel()):
                copies.append(None)
            elif reuse[i]:
                old[i].copy_(t.detach())
                copies.append(old[i])
            else:
                copies.append(t.detach().to("cpu", copy=True))
        g.copies, self.bytes = copies, total
        return None

    def drop(self, g: _Group) -> None:
        self.bytes -= self.size(g.copies)
        g.copies = None

    @staticmethod
    def differing(pairs: list, limit: int) -> Tuple[int, bool]:
        """Values of the tensors that differ from their copies, counted on the host a chunk at a time (stops past
        limit: (count so far, True))."""
        n = 0
        for t, c in pairs:
            es = min(t.element_size(), 4)
            view = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[es]
            a = t.detach().contiguous().view(-1).view(torch.uint8).view(view)
            b = c.contiguous().view(-1).view(torch.uint8).view(view)
            for lo in range(0, a.numel(), COUNT_CHUNK):
                n += int((a[lo:lo + COUNT_CHUNK].cpu() != b[lo:lo + COUNT_CHUNK]).sum())
                if n > limit:
                    return n, True
        return n, False


class WeightScan:
    """Scheduled weight integrity for one serving guard (ServeGuard.weight_scan()): poll() at each of the guard's
    reads.  budget_mb: bytes compared per read; target_age: seconds within which every weight should be compared
    again (the budget grows, up to max_mb, at the measured time between reads); repair: keep host copies and write a
    changed group back when few values changed."""

    def __init__(self, guard=None, budget_mb: float = DEFAULT_BUDGET_MB, target_age: Optional[float] = None,
                 max_mb: float = DEFAULT_MAX_MB, max_gap: float = 4.0, repair: bool = False,
                 repair_max_values: int = REPAIR_MAX_VALUES, host_allowance: Optional[int] = None):
        self.guard = guard
        self.groups: List[_Group] = []
        self.budget = max(1, int(float(budget_mb) * (1 << 20)))
        self.max_budget = max(self.budget, int(float(max_mb) * (1 << 20)))
        self.target_age = float(target_age) if target_age else None
        self.max_gap = float(max_gap)
        self.repair = bool(repair)
        self.repair_max_values = max(0, int(repair_max_values))
        self.repair_off: Optional[str] = None
        self.copies = _Copies(host_allowance)
        self.paused = False
        self.not_scanned: dict = {}
        self.events: list = []
        self._turn = 0                         # next group in the round
        self._round_began = time.monotonic()
        self._gap: Optional[float] = None      # smoothed time between reads
        self._last_read: Optional[float] = None
        self._warned_age = False
        self._taken_slots: set = set()
        self._in_flight: dict = {}             # device -> [_InFlight]
        self._repairs_due: list = []           # (group, generation, window, last clean)
        self.stats = {"entries": 0, "bytes": 0, "reads": 0, "entries_compared": 0, "bytes_compared": 0,
                      "passes": 0, "last_pass_seconds": None, "changed": 0, "alerts": 0, "references_retaken": 0,
                      "budget_bytes_now": self.budget, "target_met": None, "repaired": 0, "repair_failed": 0,
                      "host_copy_bytes": 0}

    @property
    def entries(self) -> List[_Group]:
        return self.groups

    # ---------------------------------------------------------------------------------------------- registering
    def add(self, name: str, get: Callable[[], Sequence[Optional[torch.Tensor]]], kind: str,
            module: Optional[torch.nn.Module] = None) -> Optional[int]:
        """Register a group of tensors (get() returns them as they are now) with its reference taken now; kind names
        what the tensors are ("checked", "quantized", "unchecked", "other").  The group's index, or None."""
        ts = list(get())
        live = [t for t in ts if isinstance(t, torch.Tensor) and t.numel()]
        if not live:
            self.not_scanned[name] = "no weight tensors to compare"
            return None
        g = _Group(name, get, kind, module, live[0].device, sum(t.numel() * t.element_size() for t in live))
        with torch.inference_mode(False), torch.no_grad():
            self._reference(g, ts)
        self.groups.append(g)
        self.stats["entries"] = len(self.groups)
        self.stats["bytes"] += g.nbytes
        self.not_scanned.pop(name, None)
        return len(self.groups) - 1

    def sync(self) -> None:
        """Take in the guard's checked layers registered since the last call."""
        for slot, lay in enumerate(getattr(self.guard, "layers", None) or []):
            if slot not in self._taken_slots:
                self._taken_slots.add(slot)
                m = lay["module"]
                self.add(lay["name"], lambda m=m: (getattr(m, "weight", None), _bias_of(m)), "checked", m)

    def refresh(self, module: Optional[torch.nn.Module] = None, kind: Optional[str] = None,
                name: Optional[str] = None) -> int:
        """After an intended update: new references for the selected groups (all by default), compared again from
        the next read; comparisons in flight and repairs not yet made for them are dropped."""
        chosen = [g for g in self.groups if (module is None or g.module is module) and
                  (kind is None or g.kind == kind) and (name is None or g.name == name)]
        self._in_flight.clear()
        with torch.inference_mode(False), torch.no_grad():
            for g in chosen:
                self._reference(g, g.tensors())
                g.status, g.why_out, g.clean_time, g.clean_step, g.since = (Status.PROVISIONAL, None, None, None,
                                                                            time.monotonic())
                self.not_scanned.pop(g.name, None)
        self._repairs_due = [r for r in self._repairs_due if r[1] == r[0].gen]
        return len(chosen)

    def _reference(self, g: _Group, ts: list) -> None:
        g.ref = fingerprints(ts, g.device)
        g.places, g.objects = [_where(t) for t in ts], [id(t) for t in ts]
        g.ref_step = getattr(self.guard, "_marked_step", None)
        g.gen += 1
        if g.status != Status.EXCLUDED:
            g.status = Status.PROVISIONAL
        if self.repair:
            why = self.copies.keep(g, ts)
            if why:
                self._stop_repair(why)
            self.stats["host_copy_bytes"] = self.copies.bytes

    def _stop_repair(self, why: str) -> None:
        self.repair, self.repair_off = False, why
        for g in self.groups:
            g.copies = None
        self.copies.bytes = 0
        self.stats["host_copy_bytes"] = 0
        self._repairs_due = []
        log.warning("sdcguard: weight repair is off: %s; the scan still compares and alerts", why)

    def _exclude(self, g: _Group, why: str) -> None:
        if g.status != Status.EXCLUDED:
            log.warning("sdcguard: the weight scan no longer compares %s: %s", g.name, why)
        g.status, g.why_out = Status.EXCLUDED, why
        self.not_scanned[g.name] = why
        self.copies.drop(g)
        self.stats["host_copy_bytes"] = self.copies.bytes

    def _overlap(self, g: _Group, ts: list) -> Optional[_Group]:
        """Another group one of whose tensors (a different tensor object) lives at one of ts's addresses."""
        mine = {(w[0], w[1]): id(t) for t, w in ((t, _where(t)) for t in ts) if w}
        for other in self.groups:
            if other is g:
                continue
            for w, oid in zip(other.places, other.objects):
                if w and (w[0], w[1]) in mine and mine[(w[0], w[1])] != oid:
                    return other
        return None

    # ------------------------------------------------------------------------------------------------- reading
    def poll(self, wait: bool = False) -> list:
        """Report the comparisons that came back, start the next ones (up to this read's budget), and make the
        repairs that are due."""
        self.sync()
        self.stats["reads"] += 1
        now = time.monotonic()
        if self._last_read is not None:
            gap = min(now - self._last_read, self.max_gap)
            self._gap = gap if self._gap is None else 0.8 * self._gap + 0.2 * gap
        self._last_read = now
        out = self._settle(wait)
        if self.groups and not self.paused:
            out += self._compare_next(wait)
        if self._repairs_due:
            self._repair_due()
        return out

    def target(self) -> int:
        """Bytes this read compares: the budget, or with a verification-age target enough that a pass over the live
        groups takes at most two thirds of it at the measured time between reads (at most max_mb)."""
        if not self.target_age or not self._gap:
            return self.budget
        live = sum(g.nbytes for g in self.groups if g.live())
        want = int(live * self._gap / (self.target_age * 2 / 3)) + 1
        self.stats["target_met"] = want <= self.max_budget
        if want > self.max_budget and not self._warned_age:
            self._warned_age = True
            log.warning("sdcguard: the weight scan can't compare every weight within %gs at %.2fs between reads "
                        "(it would need %.0f MB a read, above the %.0f MB most)", self.target_age, self._gap,
                        want / (1 << 20), self.max_budget / (1 << 20))
        return max(self.budget, min(want, self.max_budget))

    def oldest_age(self, now: Optional[float] = None) -> Optional[float]:
        now = time.monotonic() if now is None else now
        ages = [now - (g.clean_time if g.clean_time is not None else g.since) for g in self.groups if g.live()]
        return max(ages) if ages else None

    def _next_group(self) -> _Group:
        g = self.groups[self._turn]
        self._turn = (self._turn + 1) % len(self.groups)
        if self._turn == 0:                    # a pass over every group ended
            t = time.monotonic()
            self.stats["passes"] += 1
            self.stats["last_pass_seconds"] = round(t - self._round_began, 3)
            self._round_began = t
        return g

    def _ready(self, g: _Group) -> Optional[list]:
        """g's tensors if it is to be compared now; otherwise None, with g taken in again or left out."""
        if not g.live():
            return None
        ts = g.tensors()
        other = self._overlap(g, ts)
        if other is not None:
            self._exclude(g, f"shares its memory with {other.name}'s tensors (CPU offloading)")
            if other.status != Status.EXCLUDED:
                self._exclude(other, f"shares its memory with {g.name}'s tensors (CPU offloading)")
            return None
        if [_where(t) for t in ts] == g.places:
            return ts
        if g.status == Status.PROVISIONAL:     # never compared: the reference is taken where the tensors are now
            self._reference(g, ts)
            self.stats["references_retaken"] += 1
        else:
            self._exclude(g, "its tensors moved or changed shape after they were compared (call refresh() after an "
                             "intended reload)")
        return None

    def _compare_next(self, wait: bool) -> list:
        """Fingerprint the next groups and compare them with their references: per device one stacked comparison
        and one count per group, all on the GPU."""
        budget = self.stats["budget_bytes_now"] = self.target()
        step = getattr(self.guard, "_marked_step", None)
        picked: dict = {}
        spent = 0
        with torch.inference_mode(False), torch.no_grad():
            for _ in range(len(self.groups)):
                if spent >= budget and picked:
                    break
                g = self._next_group()
                ts = self._ready(g)
                if ts is not None:
                    picked.setdefault(g.device, []).append((g, ts))
                    spent += g.nbytes
            out = []
            for dev, items in picked.items():
                flat = [t for _, ts in items for t in ts]
                owner = torch.tensor([i for i, (_, ts) in enumerate(items) for _ in ts], dtype=torch.int64)
                if dev.type == "cuda":
                    owner = owner.pin_memory().to(dev, non_blocking=True)
                differs = (fingerprints(flat, dev) != torch.cat([g.ref for g, _ in items])).any(-1)
                flags = torch.zeros(len(items), dtype=torch.int32, device=dev).index_add_(0, owner,
                                                                                          differs.to(torch.int32))
                batch = [(g, g.gen, step) for g, _ in items]
                if dev.type == "cuda" and not wait:
                    host = torch.empty(len(items), dtype=torch.int32, pin_memory=True)
                    host.copy_(flags, non_blocking=True)
                    done = torch.cuda.Event()
                    done.record(torch.cuda.current_stream(dev))
                    self._in_flight.setdefault(dev, []).append(_InFlight(host, done, batch))
                else:
                    out += self._verdicts(flags.cpu(), batch)
                self.stats["entries_compared"] += len(batch)
                self.stats["bytes_compared"] += sum(g.nbytes for g, _ in items)
        return out

    def _settle(self, wait: bool) -> list:
        out = []
        for dev, batches in list(self._in_flight.items()):
            left = []
            for b in batches:
                if wait:
                    b.done.synchronize()
                if b.done.query():
                    out += self._verdicts(b.flags, b.groups)
                else:
                    left.append(b)
            if left:
                self._in_flight[dev] = left
            else:
                self._in_flight.pop(dev)
        return out

    def _verdicts(self, flags: torch.Tensor, batch: list) -> list:
        out = []
        now = time.monotonic()
        for differs, (g, gen, step) in zip(flags.tolist(), batch):
            if gen != g.gen or g.status == Status.EXCLUDED:   # a new reference, or left out, since it started
                continue
            g.compared += 1
            if not differs:
                g.status, g.clean_time, g.clean_step = Status.CLEAN, now, step
                continue
            if g.status == Status.CHANGED:
                continue
            g.status = Status.CHANGED
            self.stats["changed"] += 1
            ev = self._changed_event(g, now, step)
            out.append(ev)
            if self.repair and g.copies:
                self._repairs_due.append((g, g.gen, ev.extra.get("read_window_steps"),
                                          ev.extra.get("last_clean_read_steps")))
        return out

    # -------------------------------------------------------------------------------------------------- repair
    def _repair_due(self) -> None:
        """Changed groups with repair on: written back when at most repair_max_values values differ from the copy,
        then verified against the reference; a record goes out either way (the alert stands)."""
        due, self._repairs_due = self._repairs_due, []
        for g, gen, window, clean in due:
            if gen != g.gen or g.status != Status.CHANGED:
                continue
            at = getattr(self.guard, "_marked_step", None)
            counts = None
            try:
                with torch.inference_mode(False), torch.no_grad():
                    why, counts = self._write_back(g, at)
            except Exception as ex:  # noqa: BLE001  (a failed repair leaves the alert as it is)
                why = f"the restore failed: {type(ex).__name__}: {ex}"[:300]
            if why is None:
                g.status, g.repairs, g.gen = Status.CLEAN, g.repairs + 1, g.gen + 1
                g.clean_time, g.clean_step, g.compared_at_repair = time.monotonic(), at, g.compared
                self.stats["repaired"] += 1
            else:
                self.stats["repair_failed"] += 1
            self._publish(self._repair_event(g, why, at, window, clean, counts))

    def _write_back(self, g: _Group, at) -> Tuple[Optional[str], Optional[dict]]:
        """(None, counts) after a verified write-back, or (why not, counts)."""
        ts, copies = g.tensors(), g.copies or []
        if [_where(t) for t in ts] != g.places or len(copies) != len(ts):
            return "its tensors moved or changed since the clean copy was taken", None
        other = self._overlap(g, ts)
        if other is not None:
            return f"it shares its memory with {other.name}'s tensors (CPU offloading)", None
        pairs = [(t, c) for t, c in zip(ts, copies) if c is not None and isinstance(t, torch.Tensor)]
        if any(t.shape != c.shape or t.dtype != c.dtype for t, c in pairs):
            return "a tensor's shape or dtype differs from its clean copy", None
        if g.device.type == "cuda":
            torch.cuda.synchronize(g.device)
        n, stopped = _Copies.differing(pairs, self.repair_max_values)
        counts = {"values_changed": n, "values": sum(c.numel() * (2 if c.element_size() == 8 else 1) for _, c in pairs),
                  "at_least": stopped}
        if n > self.repair_max_values:
            return (f"{'at least ' if stopped else ''}{n} values differ from the copy kept with the reference, more "
                    f"than a fault in memory changes (repair writes back at most {self.repair_max_values}): an update "
                    "the guard was not told about, or a stray write"), counts
        try:
            for t, c in pairs:
                with torch.inference_mode(t.is_inference()), torch.no_grad():
                    t.copy_(c)
        finally:
            note = getattr(self.guard, "_weights_restored", None)
            if note is not None and g.module is not None:
                try:
                    note(g.module, at)
                except Exception:  # noqa: BLE001
                    pass
        if g.device.type == "cuda":
            torch.cuda.synchronize(g.device)
        if torch.equal(fingerprints(ts, g.device).cpu(), g.ref.cpu()):
            return None, counts
        return "the restored weights still don't match their reference fingerprint", counts

    # ------------------------------------------------------------------------------------------------- reports
    def _publish(self, ev) -> None:
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

    def _changed_event(self, g: _Group, now: float, step: Optional[int]):
        from .serve import SDCEvent
        window, since = None, None
        if step is not None:
            if g.clean_step is not None:
                window, since = [min(g.clean_step + 1, step), step], "the last clean comparison"
            elif g.ref_step is not None:
                window, since = [min(g.ref_step + 1, step), step], "the reference (at load or the last refresh)"
            else:
                window, since = [0, step], "load"
        detail = {"where": g.name, "finding": "weights_changed", "kind": g.kind, "weights_changed_since_load": True,
                  "recheck": {"verdict": "weights_changed",
                              "why": "the group's tensors no longer match their reference fingerprint (taken at load "
                                     "or at the last refresh)"},
                  "read_window_steps": window, "window_since": since,
                  "last_clean_read_steps": [g.clean_step, g.clean_step] if g.clean_step is not None else None,
                  "seconds_since_last_clean_comparison": (round(now - g.clean_time, 3)
                                                          if g.clean_time is not None else None),
                  "last_pass_seconds": self.stats["last_pass_seconds"],
                  "scan": {"budget_bytes": self.stats["budget_bytes_now"], "entries": len(self.groups),
                           "target_age_seconds": self.target_age},
                  "reading": "a weight bit changed after load: memory corruption, or an update the guard was not told "
                             "about (refresh() after an intended one); requests this layer served since its last "
                             "clean comparison may have used the changed weights"}
        ev = SDCEvent(detector="serve_weights", layer=g.name, z=float("inf"), extra=detail)
        self.stats["alerts"] += 1
        self._publish(ev)
        return ev

    def _repair_event(self, g: _Group, why: Optional[str], at, window, clean, counts):
        from .serve import SDCEvent
        ok = why is None
        counts = counts or {}
        start = window[0] if window else at
        detail = {"where": g.name, "kind": g.kind, "finding": "weights_restored" if ok else "weights_restore_failed",
                  "recheck": {"verdict": "weights_restored" if ok else "restore_failed",
                              "why": "the copy kept with the reference was written back and the tensors match their "
                                     "reference fingerprint again" if ok else why},
                  "repairs": g.repairs, "values_changed": counts.get("values_changed"), "values": counts.get("values"),
                  "values_changed_at_least": bool(counts.get("at_least")), "repaired_at_step": at,
                  "read_window_steps": [start, at] if start is not None and at is not None and start <= at else None,
                  "last_clean_read_steps": clean,
                  "reading": "restored in place and verified; requests this layer served from its last clean "
                             "comparison to the repair may have used the changed weights" if ok else
                             f"not restored ({why}): the layer keeps its changed weights"}
        (log.warning if ok else log.error)("sdcguard: weight repair of %s: %s", g.name,
                                           f"restored ({counts.get('values_changed')} values) and verified" if ok
                                           else why)
        return SDCEvent(detector="serve_weights", layer=g.name, z=0.0 if ok else float("inf"), extra=detail)

    def coverage(self) -> dict:
        kinds: dict = {}
        for g in self.groups:
            kinds[g.kind] = kinds.get(g.kind, 0) + 1
        age = self.oldest_age()
        return {"entries": len(self.groups), "by_kind": kinds, "bytes": self.stats["bytes"],
                "budget_bytes_per_read": self.budget, "budget_bytes_now": self.stats["budget_bytes_now"],
                "target_age_seconds": self.target_age, "target_met": self.stats["target_met"],
                "oldest_verification_age_seconds": round(age, 3) if age is not None else None,
                "oldest_within_target": (age <= self.target_age) if self.target_age and age is not None else None,
                "passes": self.stats["passes"], "last_pass_seconds": self.stats["last_pass_seconds"],
                "never_compared": sorted(g.name for g in self.groups if not g.compared and g.live()),
                "repair": {"on": self.repair, "off_because": self.repair_off, "max_values": self.repair_max_values,
                           "host_copy_bytes": self.copies.bytes, "host_allowance_bytes": self.copies.allowance,
                           "repaired": self.stats["repaired"], "failed": self.stats["repair_failed"],
                           "entries_repaired": sorted(g.name for g in self.groups if g.repairs),
                           "not_compared_since_repair": sorted(g.name for g in self.groups if g.repairs and g.live()
                                                               and g.compared <= g.compared_at_repair)},
                "changed": sorted(g.name for g in self.groups if g.status == Status.CHANGED),
                "not_scanned": dict(self.not_scanned), "kernel": "sdc_fingerprint2"}


def _bias_of(m) -> Optional[torch.Tensor]:
    b = getattr(m, "bias", None)
    return b if isinstance(b, torch.Tensor) else None
