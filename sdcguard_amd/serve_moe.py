"""Checks of fused MoE experts in serving: a sampled exact recompute of the routed experts' output (reference:
serve_moe.py).

A fused MoE layer computes, for each token x and its top-k experts e_k with routing weights g_k,
y = sum_k g_k W2_e (act(W1_e x) * (W3_e x)) for all experts in one kernel, so no single matmul can be checked by a
checksum from outside.  At each model step one MoE layer (the layer whose index is the step modulo the number of MoE
layers) recomputes the output of SAMPLES rows of its batch from its own input, routing and weights, with the fused
kernel's roundings (the first matmul in fp32 rounded to bf16/fp16, the activation rounded, the product rounded, the
second matmul in fp32 times the routing weight rounded, the experts summed in fp32), and scores each output in units
of   u |r| + OUT_FLIPS 2u max_k |c_k| + KAPPA u sqrt(sum_k g_k^2 sum_i (W2_ni h_i)^2) + FLIPS max_k,i |g_k W2_ni| s_i
(u the dtype's unit roundoff; s_i the size of a rounding flip of h_i or its inputs); over MOE_Z is an alarm.  Rows are
drawn from the step's real rows when known; a row whose experts are all -1 (a padding row of a captured batch) isn't
judged.  The layer also reads the expert ids of every known real row: a real row with all or some experts -1 is
wrong whatever the numbers (a router fault, a corrupted id, a padding mask over a real row).

The arithmetic runs in the HIP library (moe_check.hip, sdc_moe_check): four launches that return at once unless the
layer is the active one, no host synchronisation, no memory set (graph-safe).  What it sees: wrong experts, another
row's output, wrong scaling, non-finite values, large bit errors.  Not a weight changed in memory (both sides read
the same weights; an alert says whether the weights changed since load), quantized experts, experts with biases,
activations other than gated SiLU/GELU, or layers that combine across GPUs.
"""
from __future__ import annotations

import math
import struct
import threading
from typing import Optional

import torch

from .serve import SDCEvent

MOE_Z = 6.0
SAMPLES = 2
KAPPA = 1.0
FLIPS = 1.0
OUT_FLIPS = 2.0
MOE_SCHEMA = 1
COLS = 11
C_ROW, C_COL, C_OUT, C_REF, C_STEP, C_CALLS, C_ROWS, C_UNJ, C_UNROUTED, C_PARTIAL, C_BADROW = range(COLS)
CAP_COLS = 4                     # claimed, row, step, score bits
M32 = 0xFFFFFFFF
ROW_A, ROW_B = 7919, 104729
ROWS_SHIFT = 32
ROWS_MAX = (1 << 31) - 1
ACT = {"silu": 0, "gelu": 1}
PLACE_KEPT = "the kept row's worst output, rechecked"
PLACE_MAXIMA = "the read's score maxima (row, column and values of the worst score)"


def _f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", int(bits) & M32))[0]


def dtype_consts(dtype: torch.dtype) -> tuple:
    """(unit roundoff, subnormal spacing, largest finite value) of the output dtype (bf16's spacing is a small
    normal fp32 value, so 0 / spacing stays 0 where fp32 subnormals are flushed)."""
    if dtype == torch.float16:
        return 2.0 ** -11, 2.0 ** -24, 65504.0
    if dtype == torch.bfloat16:
        return 2.0 ** -8, 1e-37, float(torch.finfo(torch.bfloat16).max)
    return 2.0 ** -8, 1e-37, float(torch.finfo(torch.float32).max)


def sample_rows(step: torch.Tensor, m, device, nlayers: int = 1) -> torch.Tensor:
    """The rows a layer's check takes at a step: from the layer's own turn count (step // nlayers), of its first m
    rows (an int, or a tensor for the step's real rows)."""
    j = torch.arange(SAMPLES, device=device, dtype=torch.int64)
    mm = m.clamp(min=1) if isinstance(m, torch.Tensor) else max(int(m), 1)
    return (torch.div(step, max(int(nlayers), 1), rounding_mode="floor") * ROW_A + j * ROW_B) % mm


def rows_of(raw: torch.Tensor, m: int) -> torch.Tensor:
    """The rows a step's samples come from: its real rows packed in the step buffer when known, else all m."""
    real = (raw >> ROWS_SHIFT) & ROWS_MAX
    return torch.where(real > 0, real.clamp(max=m), torch.full_like(real, m))


def pack_step(step: int, rows: Optional[int] = None) -> int:
    """The step buffer's value: the step (low 32 bits) and, above it, the step's real rows (0: unknown)."""
    r = int(rows) if rows is not None and int(rows) > 0 else 0
    return (min(r, ROWS_MAX) << ROWS_SHIFT) | (int(step) & M32)


def _code(dt: torch.dtype) -> int:
    return {torch.bfloat16: 0, torch.float16: 1, torch.float32: 4}[dt]


def moe_check(x: torch.Tensor, out: torch.Tensor, topk_w: torch.Tensor, topk_ids: torch.Tensor, w13: torch.Tensor,
              w2: torch.Tensor, expert_map: Optional[torch.Tensor], act: int, routed_first: bool, state: torch.Tensor,
              slot: int, stepbuf: torch.Tensor, nlayers: int, index: int, cap_meta: torch.Tensor, cap_x: torch.Tensor,
              cap_y: torch.Tensor, cap_ids: torch.Tensor, cap_g: torch.Tensor, line: float,
              scores_out: Optional[torch.Tensor] = None) -> None:
    """One call's check queued on the GPU (serve_moe.py:185-258).  x, out: [rows, H]; topk_w, topk_ids: [rows, k];
    w13 [E, 2I, H], w2 [E, H, I]; state[slot] the layer's COLS counters; cap_* its kept row; stepbuf[0] the packed
    step.  Only the active layer's call computes anything."""
    from . import _lib
    m, hdim = x.shape[0], x.shape[-1]
    if m == 0:
        return
    _lib.require_gpu(x, out, topk_w, topk_ids, w13, w2, state, stepbuf)
    x2, y2 = x.reshape(m, hdim), out.reshape(m, hdim)
    x2 = x2 if x2.stride(-1) == 1 else x2.contiguous()
    y2 = y2 if y2.stride(-1) == 1 else y2.contiguous()
    ids = topk_ids.reshape(m, -1)
    ids = ids if ids.dtype == torch.int32 and ids.is_contiguous() else ids.to(torch.int32).contiguous()
    gw = topk_w.reshape(m, -1)
    gw = gw if gw.dtype in (torch.bfloat16, torch.float16, torch.float32) else gw.float()
    gw = gw.contiguous()
    emap = None
    if expert_map is not None:
        emap = expert_map if expert_map.dtype == torch.int32 else expert_map.to(torch.int32)
    k = ids.shape[1]
    if w13.stride(-1) != 1 or w2.stride(-1) != 1:
        raise ValueError("expert weights must be contiguous along their last dimension")
    u, sp, fm = dtype_consts(out.dtype)
    L = _lib.lib()
    ws_bytes = int(L.sdc_moe_check_workspace(hdim, w2.shape[2], k))
    ws = _lib.workspace(x.device, ws_bytes)
    rc = L.sdc_moe_check(_code(out.dtype), x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0), gw.data_ptr(),
                         _code(gw.dtype), ids.data_ptr(), w13.data_ptr(), w13.stride(0), w13.stride(1), w2.data_ptr(),
                         w2.stride(0), w2.stride(1), None if emap is None else emap.data_ptr(), w13.shape[0],
                         0 if emap is None else emap.numel(), m, hdim, w2.shape[2], k,
                         int(act), int(bool(routed_first)), stepbuf.data_ptr(), max(int(nlayers), 1), int(index),
                         float(u), float(sp), float(fm), float(line), state[slot].data_ptr(), cap_meta[slot].data_ptr(),
                         cap_x[slot].data_ptr(), cap_y[slot].data_ptr(), cap_ids[slot].data_ptr(),
                         cap_g[slot].data_ptr(), None if scores_out is None else scores_out.data_ptr(),
                         ws.data_ptr(), ws_bytes, _lib.stream_of(x))
    _lib.check(rc, "sdc_moe_check")


moe_check_torch = moe_check          # the reference's names for the same call
moe_check_any = moe_check

_lib_lock = threading.Lock()
_OP = [None]


def moe_op():
    """sdcguard::moe_check, registered once (for callers under torch.compile)."""
    with _lib_lock:
        if _OP[0] is None:
            try:
                @torch.library.custom_op("sdcguard::moe_check",
                                         mutates_args=("state", "cap_meta", "cap_x", "cap_y", "cap_ids", "cap_g"))
                def _moe_check(x: torch.Tensor, out: torch.Tensor, topk_w: torch.Tensor, topk_ids: torch.Tensor,
                               w13: torch.Tensor, w2: torch.Tensor, expert_map: Optional[torch.Tensor], act: int,
                               routed_first: bool, state: torch.Tensor, slot: int, stepbuf: torch.Tensor,
                               nlayers: int, index: int, cap_meta: torch.Tensor, cap_x: torch.Tensor,
                               cap_y: torch.Tensor, cap_ids: torch.Tensor, cap_g: torch.Tensor, line: float) -> None:
                    moe_check(x, out, topk_w, topk_ids, w13, w2, expert_map, act, routed_first, state, slot, stepbuf,
                              nlayers, index, cap_meta, cap_x, cap_y, cap_ids, cap_g, line)

                @_moe_check.register_fake
                def _(*a):
                    return None

                _OP[0] = torch.ops.sdcguard.moe_check
            except (AttributeError, RuntimeError):
                _OP[0] = getattr(getattr(torch.ops, "sdcguard", None), "moe_check", None) or moe_check
        return _OP[0]


def check_call(args: tuple, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor, out) -> None:
    """Check one call of a registered MoE layer from its input, routing and (finalized) output."""
    if not isinstance(out, torch.Tensor) or not isinstance(x, torch.Tensor) or out.shape[-1] != x.shape[-1] or \
            out.shape[0] != x.shape[0]:
        return
    w13, w2, emap, act, rf, st, slot, sb, nl, idx, cm, cx, cy, ci, cg, line = args
    call = (x, out, topk_weights, topk_ids, w13, w2, emap, act, rf, st, slot, sb, nl, idx, cm, cx, cy, ci, cg, line)
    if torch.compiler.is_compiling():
        (_OP[0] if _OP[0] is not None else moe_op())(*call)
    else:
        with torch.no_grad():
            moe_check(*call)


def recheck(x_row: torch.Tensor, y_row: torch.Tensor, ids: torch.Tensor, g: torch.Tensor, w13: torch.Tensor,
            w2: torch.Tensor, expert_map: Optional[torch.Tensor], act: int, routed_first: bool, dtype: torch.dtype,
            line: float = MOE_Z) -> dict:
    """The kept row checked again, alone, with the same kernels and the experts' weights as the layer holds them now
    (every output's score; the worst one's place and values)."""
    dev = w13.device
    used = sorted({int(v) for v in (expert_map.long()[ids.long().clamp(min=0)] if expert_map is not None
                                     else ids.long()).tolist() if v >= 0})
    if not used or any(int(v) >= 0 and (expert_map is not None and int(expert_map[int(v)]) < 0)
                       for v in ids.tolist()):
        return {"verdict": "not_rechecked", "why": "the kept row's experts aren't on this GPU"}
    h = x_row.numel()
    k = ids.numel()
    x1 = x_row.reshape(1, h).to(dev, dtype)
    y1 = y_row.reshape(1, h).to(dev).to(dtype)
    st = torch.zeros(1, COLS, dtype=torch.int64, device=dev)
    cm = torch.zeros(1, CAP_COLS, dtype=torch.int32, device=dev)
    cx, cy = torch.zeros(1, h, device=dev), torch.zeros(1, h, device=dev)
    ci, cg = torch.zeros(1, max(k, 1), dtype=torch.int64, device=dev), torch.zeros(1, max(k, 1), device=dev)
    sb = torch.full((1,), pack_step(0, 1), dtype=torch.int64, device=dev)
    zs = torch.zeros(SAMPLES, h, device=dev)
    moe_check(x1, y1, g.reshape(1, k).to(dev).float(), ids.reshape(1, k).to(dev), w13, w2, expert_map, act,
              routed_first, st, 0, sb, 1, 0, cm, cx, cy, ci, cg, line, scores_out=zs)
    z = zs[0].cpu()
    keys = st[0].cpu().tolist()
    worst = _f32(keys[C_ROW] >> 32)
    bad = int((z > line).sum())
    out = {"worst_score": worst, "outputs_over_line": bad, "outputs": h, "experts": used}
    if worst > 0:
        out.update(col=keys[C_COL] & M32, output=_f32(keys[C_OUT]), expected=_f32(keys[C_REF]))
    if bad:
        return {**out, "verdict": "output_wrong",
                "why": f"{bad} of {h} outputs of the kept row are farther from the recompute (the layer's current "
                       "weights, the kept input and routing) than its rounding allows"}
    return {**out, "verdict": "output_agrees",
            "why": "the recompute of the kept row alone agrees with its output: the check disagreed when the row "
                   "ran in its batch, or the weights changed back since"}


# ------------------------------------------------------------------------------------------------- the MoE layers
def describe(mod) -> tuple:
    """(what the check needs, or None; why not) for a serving stack's fused MoE layer: unquantized bf16/fp16 experts
    on the Triton MoE kernel, no biases, a gated SiLU or GELU, nothing combined across GPUs (serve_moe.py:709-748)."""
    qm = getattr(mod, "quant_method", None)
    if type(qm).__name__ != "UnquantizedFusedMoEMethod":
        return None, f"{type(qm).__name__ if qm is not None else 'no quant method'}: quantized or another method"
    pc = getattr(getattr(mod, "moe_config", None), "moe_parallel_config", None)
    try:
        across = bool(getattr(pc, "use_all2all_kernels", False) or getattr(pc, "use_passthrough_all2all", False) or
                      int(getattr(pc, "dp_size", 1) or 1) > 1 or int(getattr(pc, "pcp_size", 1) or 1) > 1)
    except Exception:  # noqa: BLE001
        across = True
    if across:
        return None, ("expert parallelism's all-to-all, data parallelism or prefill context parallelism: the layer's "
                      "rows or output combine other GPUs', which the recompute can't read")
    backend = getattr(getattr(qm, "unquantized_backend", None), "name", None)
    if backend != "TRITON":
        return None, f"the {backend or 'unknown'} MoE backend (only the Triton MoE kernel's rounding is modelled)"
    w13, w2 = getattr(mod, "w13_weight", None), getattr(mod, "w2_weight", None)
    if not (isinstance(w13, torch.Tensor) and isinstance(w2, torch.Tensor) and w13.dim() == 3 and w2.dim() == 3):
        return None, "no expert weights the check knows"
    if w13.dtype not in (torch.bfloat16, torch.float16) or w2.dtype != w13.dtype:
        return None, f"expert weights in {w13.dtype}"
    if w13.shape[0] != w2.shape[0] or w13.shape[2] != w2.shape[1] or w13.shape[1] != 2 * w2.shape[2]:
        return None, f"expert weight shapes {tuple(w13.shape)} and {tuple(w2.shape)} aren't gate-up and down"
    if w13.shape[2] > 8192:
        return None, f"hidden size {w13.shape[2]} (at most 8192)"
    if any(isinstance(getattr(mod, b, None), torch.Tensor) for b in ("w13_bias", "w2_bias")):
        return None, "experts with biases"
    act = getattr(getattr(mod, "activation", None), "value", getattr(mod, "activation", None))
    if str(act) not in ACT:
        return None, f"activation {act}"
    if not w13.is_cuda:
        return None, "not on a GPU"
    if getattr(mod, "_sdcguard_moe", None) is not None:
        return None, "already checked by another ServeGuard"
    return {"act": ACT[str(act)], "routed_first": bool(getattr(mod, "apply_router_weight_on_input", False)),
            "top_k": int(getattr(mod, "top_k", 0) or 0)}, None


class MoEChecks:
    """The fused MoE layers one serving guard checks: add() each, finalize() once before capture, mark_step() before
    each model step (it decides which layer is active) and end_step() after, poll() with the guard's reads."""

    def __init__(self, guard=None, line: float = MOE_Z):
        line = float(line)
        if not 5.0 <= line < float("inf"):
            raise ValueError(f"the MoE check's line must be at least 5, not {line!r}")
        self.guard, self.line = guard, line
        self.layers: list = []
        self.unsupported: dict = {}
        self._state, self._cap, self._step, self._host, self._read_from = {}, {}, {}, {}, {}
        self._marked: Optional[int] = None
        self._last_clean: dict = {}
        self.worst_seen: dict = {}
        self.checks_seen: dict = {}
        self.events: list = []
        self.finalized = False
        self.stats = {"layers": 0, "active_calls": 0, "rows_checked": 0, "unjudged_outputs": 0,
                      "unrouted_real_rows": 0, "partly_routed_real_rows": 0, "alerts": 0}

    def add(self, mod, name: str) -> Optional[int]:
        if self.finalized:
            raise RuntimeError("MoE layers are added before finalize()")
        info, why = describe(mod)
        if why:
            self.unsupported[name] = why
            return None
        with torch.inference_mode(False), torch.no_grad():
            sums = (mod.w13_weight.detach().float().sum(1), mod.w2_weight.detach().float().sum(2))
        self.layers.append({"name": name, "module": mod, "device": mod.w13_weight.device, "sums": sums, **info,
                            "h": int(mod.w13_weight.shape[2]), "i": int(mod.w2_weight.shape[2])})
        self.stats["layers"] += 1
        return len(self.layers) - 1

    def finalize(self) -> int:
        """Allocate the state rows, the kept rows and the kernels' workspace on each device (before any graph is
        captured), number the layers' turns and register the op."""
        if self.finalized:
            return len(self.layers)
        from . import _lib
        by_dev: dict = {}
        for lay in self.layers:
            by_dev.setdefault(lay["device"], []).append(lay)
        n = len(self.layers)
        for dev, lays in by_dev.items():
            hmax = max(lay["h"] for lay in lays)
            kmax = max(max(lay["top_k"], 1) for lay in lays)
            for i, lay in enumerate(lays):
                lay["index"], lay["nlayers"] = i, len(lays)
            with torch.inference_mode(False):
                self._state[dev] = torch.zeros(n, COLS, dtype=torch.int64, device=dev)
                self._cap[dev] = (torch.zeros(n, CAP_COLS, dtype=torch.int32, device=dev),
                                  torch.zeros(n, hmax, device=dev), torch.zeros(n, hmax, device=dev),
                                  torch.zeros(n, max(kmax, 64), dtype=torch.int64, device=dev),
                                  torch.zeros(n, max(kmax, 64), device=dev))
                self._step[dev] = torch.zeros(1, dtype=torch.int64, device=dev)
            need = max(int(_lib.lib().sdc_moe_check_workspace(lay["h"], lay["i"], max(lay["top_k"], 1)))
                       for lay in lays)
            _lib.workspace(dev, need)
        moe_op()
        for slot, lay in enumerate(self.layers):
            lay["module"]._sdcguard_moe = self.args(slot)
        self.finalized = True
        return n

    def args(self, slot: int) -> tuple:
        lay = self.layers[slot]
        mod, dev = lay["module"], lay["device"]
        cm, cx, cy, ci, cg = self._cap[dev]
        return (mod.w13_weight, mod.w2_weight, getattr(mod, "expert_map", None), lay["act"], lay["routed_first"],
                self._state[dev], slot, self._step[dev], lay["nlayers"], lay["index"], cm, cx, cy, ci, cg, self.line)

    def refresh(self) -> int:
        """Take the experts' current weights as theirs (after an intended update)."""
        with torch.inference_mode(False), torch.no_grad():
            for lay in self.layers:
                mod = lay["module"]
                lay["sums"] = (mod.w13_weight.detach().float().sum(1), mod.w2_weight.detach().float().sum(2))
                lay.pop("restored", None)
        return len(self.layers)

    def weights_restored(self, module, step) -> None:
        """The weight scan's repair wrote these experts' load-time weights back after `step`."""
        for lay in self.layers:
            if lay["module"] is module:
                lay["restored"] = {"step": step}

    def detach(self) -> None:
        try:
            if self.layers and self.finalized:
                self.poll(wait=True)
        finally:
            for lay in self.layers:
                lay["module"].__dict__.pop("_sdcguard_moe", None)
            self.layers.clear()
            for d in (self._state, self._cap, self._step, self._host, self._read_from):
                d.clear()
            self.finalized = False

    def mark_step(self, step: int, rows: Optional[int] = None) -> None:
        """Before a model step: its number and, when known, its real rows before padding."""
        step = int(step) & M32
        self._marked = step
        for dev, sb in self._step.items():
            sb.fill_(pack_step(step, rows))
            self._read_from.setdefault(dev, step)

    def end_step(self) -> None:
        """After a model step: runs before the next one (warm-up, capture) are checked over all their rows."""
        if self._marked is None:
            return
        for sb in self._step.values():
            sb.fill_(pack_step(self._marked))

    def _window(self, dev):
        if self._marked is None:
            return None
        a = self._read_from.pop(dev, None)
        return [a if a is not None else self._marked, self._marked]

    def poll(self, wait: bool = False) -> list:
        """The counters and kept rows read back (cleared on the device); without wait, the copy started now is
        reported by a later poll."""
        events = []
        for dev, st in self._state.items():
            cm = self._cap[dev][0]
            if wait:
                pend = self._host.pop(dev, None)
                if pend is not None:
                    pend[2].synchronize()
                    events += self._report(dev, pend[0], pend[1], pend[3])
                host, hcap = st.to("cpu", copy=True), cm.to("cpu", copy=True)
                st.zero_()
                events += self._report(dev, host, hcap, self._window(dev))
                continue
            pend = self._host.get(dev)
            if pend is not None and pend[2].query():
                events += self._report(dev, pend[0], pend[1], pend[3])
                pend = None
                self._host.pop(dev, None)
            if pend is None:
                hs = torch.empty(st.shape, dtype=st.dtype, pin_memory=True)
                hc = torch.empty(cm.shape, dtype=cm.dtype, pin_memory=True)
                hs.copy_(st, non_blocking=True)
                hc.copy_(cm, non_blocking=True)
                st.zero_()
                ev = torch.cuda.Event()
                ev.record(torch.cuda.current_stream(dev))
                self._host[dev] = (hs, hc, ev, self._window(dev))
        return events

    def coverage(self) -> dict:
        return {"layers": len(self.layers), "active_calls": self.stats["active_calls"],
                "layers_checked": sum(self.checks_seen.get(lay["name"], 0) > 0 for lay in self.layers),
                "never_checked": sorted(lay["name"] for lay in self.layers if not self.checks_seen.get(lay["name"])),
                "not_attached": dict(self.unsupported), "samples_per_step": SAMPLES}

    def _report(self, dev, host, hcap, window) -> list:
        out = []
        for slot, lay in enumerate(self.layers):
            if lay["device"] != dev or slot >= host.shape[0]:
                continue
            keys = [int(v) for v in host[slot].tolist()]
            self.stats["active_calls"] += keys[C_CALLS]
            self.stats["rows_checked"] += keys[C_ROWS]
            self.stats["unjudged_outputs"] += keys[C_UNJ]
            self.stats["unrouted_real_rows"] += keys[C_UNROUTED]
            self.stats["partly_routed_real_rows"] += keys[C_PARTIAL]
            self.checks_seen[lay["name"]] = self.checks_seen.get(lay["name"], 0) + keys[C_CALLS]
            routed_ok = not (keys[C_UNROUTED] or keys[C_PARTIAL])
            if not routed_ok:
                out.append(self._route_alert(slot, keys, window))
            z = _f32(keys[C_ROW] >> 32)
            self.worst_seen[lay["name"]] = max(self.worst_seen.get(lay["name"], 0.0), z)
            if not (z > self.line):
                if keys[C_CALLS] and window is not None and routed_ok:
                    self._last_clean[lay["name"]] = list(window)
                continue
            out.append(self._alert(dev, slot, keys, [int(v) for v in hcap[slot].tolist()], window, z))
        return out

    def _emit(self, lay, z: float, detail: dict) -> SDCEvent:
        ev = SDCEvent(detector="serve_moe", layer=lay["name"], z=z, row=detail.get("row"), extra=detail)
        self.stats["alerts"] += 1
        self.events.append(ev)
        g = self.guard
        if g is not None and getattr(g, "on_alert", None):
            try:
                g.on_alert(ev)
            except Exception:  # noqa: BLE001  (an alert callback never breaks serving)
                pass
        return ev

    def _route_alert(self, slot, keys, window) -> SDCEvent:
        lay = self.layers[slot]
        none_, some = keys[C_UNROUTED], keys[C_PARTIAL]
        last = (keys[C_BADROW] & M32) - 1
        step = (keys[C_BADROW] >> 32) & M32
        detail = {"where": lay["name"], "kind": "moe_routing",
                  "finding": "real_rows_unrouted" if none_ else "real_rows_partly_routed",
                  "real_rows_without_experts": none_, "real_rows_missing_some_experts": some,
                  "row": last if last >= 0 else None,
                  "captured": {"row": last, "step": step if self._marked is not None else None} if last >= 0 else None,
                  "recheck": {"verdict": "output_wrong",
                              "why": "a real token's row had expert ids of -1 (every real token gets top_k experts; "
                                     "-1 is for padding rows), so the layer's output for it isn't its experts' sum"},
                  "read_window_steps": window, "last_clean_read_steps": self._last_clean.get(lay["name"]),
                  "reading": "a real row reached the experts with no expert (or some missing): a router fault, a "
                             "corrupted expert id, or a padding mask that marked a real row"}
        return self._emit(lay, math.inf, detail)

    def _alert(self, dev, slot, keys, cap, window, z) -> SDCEvent:
        lay = self.layers[slot]
        mod = lay["module"]
        dtype = mod.w13_weight.dtype
        captured, rc = None, None
        if cap[0]:
            cm, cx, cy, ci, cg = self._cap[dev]
            h, k = lay["h"], max(lay["top_k"], 1)
            x_row, y_row = cx[slot, :h].clone(), cy[slot, :h].clone()
            ids, gw = ci[slot, :k].clone(), cg[slot, :k].clone()
            cm[slot].zero_()
            captured = {"row": cap[1] & M32, "step": (cap[2] & M32) if self._marked is not None else None,
                        "score": _f32(cap[3]), "experts": ids.tolist(), "weights": gw.tolist()}
            try:
                rc = recheck(x_row, y_row, ids.to(torch.int32), gw, mod.w13_weight, mod.w2_weight,
                             getattr(mod, "expert_map", None), lay["act"], lay["routed_first"], dtype, self.line)
            except Exception as e:  # noqa: BLE001  (diagnosis is best effort)
                rc = {"verdict": "not_rechecked", "why": f"{type(e).__name__}: {e}"}
        changed = None
        try:
            with torch.no_grad():
                now = (mod.w13_weight.detach().float().sum(1), mod.w2_weight.detach().float().sum(2))
            changed = not (torch.equal(now[0], lay["sums"][0]) and torch.equal(now[1], lay["sums"][1]))
        except Exception:  # noqa: BLE001
            pass
        if rc is not None and rc.get("verdict") == "output_agrees" and changed:
            rc = {**rc, "verdict": "weights_changed",
                  "why": "the kept row agrees with a recompute from the experts' current weights, which differ from "
                         "their weights at load: the weights changed in memory (refresh() after an intended update)"}
        if rc is not None and captured is not None:
            from .serve_weights import before_repair, repair_why
            if before_repair(lay.get("restored"), captured["step"]):
                rc = {**rc, "verdict": "unknown", "why": repair_why(lay["restored"], captured["step"])}
        yv, rv = _f32(keys[C_OUT]), _f32(keys[C_REF])
        row, col, place = keys[C_ROW] & M32, keys[C_COL] & M32, PLACE_MAXIMA
        if captured is not None and rc is not None and rc.get("outputs_over_line") and rc.get("col") is not None:
            row, col, yv, rv, place = captured["row"], rc["col"], rc["output"], rc["expected"], PLACE_KEPT
        u = dtype_consts(dtype)[0]
        detail = {"where": lay["name"], "kind": "moe_experts", "max_z": z, "row": row, "col": col, "output": yv,
                  "expected": rv, "place": place,
                  "relative_error": (abs(yv - rv) / abs(rv)) if rv and rv == rv else None, "captured": captured,
                  "recheck": rc or {"verdict": "not_rechecked",
                                    "why": "no row was kept for this alert (the layer's kept row was taken by an "
                                           "earlier alert that hasn't been read yet)"},
                  "weights_changed_since_load": changed, "read_window_steps": window,
                  "last_clean_read_steps": self._last_clean.get(lay["name"]),
                  "check_config": {"line": self.line, "samples_per_step": SAMPLES, "kappa": KAPPA, "flips": FLIPS,
                                   "unit_roundoff": u,
                                   "reference": "sampled recompute with the fused MoE kernel's rounding steps"},
                  "reading": "an output of the layer's routed experts differs from a recompute from the layer's own "
                             "input, routing and weights by more than the kernel's rounding allows"}
        return self._emit(lay, z, detail)
