"""Checks of FP8 quantization in serving (reference: serve_fp8.py): were a layer's FP8 inputs and their scale made
from this step's own rows, by the recipe the layer runs?

FP8 layers quantize their bf16/fp16 input to FP8 E4M3 right before the GEMM with a scale that is fixed (static) or
computed from the input (dynamic: one per row, max |x| / 448 and at least 1 / (448 * 512), or one for the whole
input, max |x| / 448).  A step's input is padded to a graph's batch size, and the padding rows hold what an earlier
step left there: a per-tensor scale taken over them makes a request's answer depend on the request before it.  At
each call the check recomputes, from the step's real rows only (published on the device by mark_step and cleared by
end_step, so warm-up and capture runs are not judged):
  - the scale: per tensor, max |x| over the real rows / 448 against the scale the GEMM got (a scale equal to the
    maximum over every row, padding included, is reported as taken from rows outside the batch); per token, the
    scale of SAMPLES real rows, each its own;
  - the FP8 values of SAMPLES real rows quantized with the scale the GEMM got, as the layer's kernels do, against
    the codes the GEMM got: two or more FP8 steps apart is an alarm, one step is counted (fast-math kernels).
Static scales are weights: they are compared with their value at load.  The arithmetic runs in the HIP library
(fp8_quant.hip, sdc_fp8_quant_check): no host synchronisation and no memory set, so a captured graph can hold it.
"""
from __future__ import annotations

import struct
import threading
from typing import Optional

import torch

from .serve import SDCEvent

FP8_MAX = 448.0
MIN_SCALE = 1.0 / (448.0 * 512.0)
SAMPLES = 2
SCALE_TOL = 2.0 ** -8          # relative: one bf16 rounding (a compiled graph may quantize the unrounded fp32 norm)
RECIPES = {"static": 0, "dynamic_tensor": 1, "dynamic_token": 2}
ROW_A, ROW_B = 7919, 104729
M32 = 0xFFFFFFFF
S31 = 0x7FFFFFFF
COLS = 8
# state row: calls judged, calls with a wrong scale, of them taken from outside rows, sampled rows with a value two
# or more steps off, values one step off, last finding ((step & S31) << 32 | kind << 24 | row), worst scale ratio
# bits, static scale changed (serve_fp8.py:46-50)
C_CALLS, C_SCALE, C_OUTSIDE, C_VALUES, C_ONE, C_LAST, C_RATIO, C_STATIC = range(COLS)
KIND_SCALE, KIND_OUTSIDE, KIND_VALUES, KIND_STATIC = 1, 2, 3, 4
EVERY_ROW = 0xFFFFFF
_DT_F32 = 4


def _f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", int(bits) & M32))[0]


def unwrap31(s31: int, marked: Optional[int]) -> int:
    """The step whose low 31 bits are s31, at or before the step marked last (steps are 32-bit)."""
    s31 = int(s31) & S31
    if marked is None:
        return s31
    s = (int(marked) & ~S31 & M32) | s31
    if s > int(marked):
        s -= 1 << 31
    return s if s >= 0 else s31


def fp8_order(codes: torch.Tensor) -> torch.Tensor:
    """FP8 E4M3 codes (uint8) as integers in the order of the values they encode (one representable step = 1;
    +0 and -0 both 0)."""
    c = codes.to(torch.int32)
    mag = c & 0x7F
    return torch.where((c & 0x80) != 0, -mag, mag)


def quantize(x_rows: torch.Tensor, scale: torch.Tensor, divide: bool) -> torch.Tensor:
    """FP8 quantization of some rows with their scale as the layers' kernels do it, as uint8 codes (a utility for
    making inputs; the check itself runs in the library)."""
    xf = x_rows.float()
    s = scale.float()
    v = xf / s if divide else xf * (1.0 / s)
    return v.clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn).view(torch.uint8)


def sample_rows(step: torch.Tensor, real: torch.Tensor) -> torch.Tensor:
    """The rows a call samples: (step * 7919 + j * 104729) % rows, j < SAMPLES."""
    j = torch.arange(SAMPLES, device=real.device, dtype=torch.int64)
    return (step * ROW_A + j * ROW_B) % real.clamp(min=1)


def _dtype_code(dt: torch.dtype) -> int:
    from . import _lib
    return _DT_F32 if dt == torch.float32 else _lib.dtype_code(dt)


def quant_check(x2: torch.Tensor, xq: torch.Tensor, xs: torch.Tensor, recipe: int, scale_ub: Optional[torch.Tensor],
                static_ref: Optional[torch.Tensor], rows_buf: torch.Tensor, stepbuf: torch.Tensor,
                state: torch.Tensor, slot: int, mult: int = 1) -> None:
    """One call's check, queued on the GPU (serve_fp8.py:79-178).  x2: [M, K] the layer's input (bf16, fp16 or
    fp32); xq: [M', K] (M' >= M) the FP8 input the GEMM got (float8_e4m3fn or its uint8 codes); xs: its scale(s),
    fp32; rows_buf[0]: the step's real rows (0: nothing judged); stepbuf[0]: the step; state[slot]: the layer's
    COLS int64 counters; mult: input rows per token (an MoE layer's second quantization has top_k)."""
    from . import _lib
    m, k = x2.shape
    if m == 0 or k == 0:
        return
    _lib.require_gpu(x2, xq, xs, rows_buf, stepbuf, state)
    q = xq.view(torch.uint8) if xq.dtype != torch.uint8 else xq
    s = xs.reshape(-1)
    if s.dtype != torch.float32:
        s = s.float()
    row = state[slot]
    if row.dtype != torch.int64 or row.numel() < COLS or row.stride(0) != 1:
        raise ValueError("state rows are int64 with COLS contiguous counters")
    ub = None if scale_ub is None else scale_ub.reshape(-1)[:1].float()
    ref = None if static_ref is None else static_ref.reshape(-1)[:1].float()
    L = _lib.lib()
    ws_bytes = int(L.sdc_fp8_quant_check_workspace(m))
    ws = _lib.workspace(x2.device, ws_bytes)
    rc = L.sdc_fp8_quant_check(_dtype_code(x2.dtype), x2.data_ptr(), x2.stride(0), x2.stride(1), m, k, q.data_ptr(),
                               q.stride(0), q.stride(1), q.shape[0], s.data_ptr(), s.numel(), s.stride(0),
                               int(recipe), None if ub is None else ub.data_ptr(),
                               None if ref is None else ref.data_ptr(), rows_buf.data_ptr(), stepbuf.data_ptr(),
                               max(int(mult), 1), row.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(x2))
    _lib.check(rc, "sdc_fp8_quant_check")


quant_check_torch = quant_check         # the reference's name for the same call

_lib_lock = threading.Lock()
_OP = [None]


def quant_op():
    """sdcguard::fp8_quant_check, registered once: one opaque op under torch.compile (serve_fp8.py:181-205)."""
    with _lib_lock:
        if _OP[0] is None:
            try:
                @torch.library.custom_op("sdcguard::fp8_quant_check", mutates_args=("state",))
                def fp8_quant_check(x2: torch.Tensor, xq: torch.Tensor, xs: torch.Tensor, recipe: int,
                                    scale_ub: Optional[torch.Tensor], static_ref: Optional[torch.Tensor],
                                    rows_buf: torch.Tensor, stepbuf: torch.Tensor, state: torch.Tensor,
                                    slot: int, mult: int) -> None:
                    quant_check(x2, xq, xs, recipe, scale_ub, static_ref, rows_buf, stepbuf, state, slot, mult)

                @fp8_quant_check.register_fake
                def _(*a):
                    return None

                _OP[0] = torch.ops.sdcguard.fp8_quant_check
            except (AttributeError, RuntimeError):
                _OP[0] = getattr(getattr(torch.ops, "sdcguard", None), "fp8_quant_check", None) or quant_check
        return _OP[0]


def check_call(args: tuple, x2: torch.Tensor, xq: torch.Tensor, xs: torch.Tensor,
               scale_ub: Optional[torch.Tensor] = None, mult: int = 1) -> None:
    """One quantization of a registered layer: its input, the FP8 input the GEMM got and its scale
    (serve_fp8.py:208-219)."""
    recipe, static_ref, rows_buf, stepbuf, state, slot = args
    if not (isinstance(xq, torch.Tensor) and isinstance(xs, torch.Tensor)) or xq.dim() != 2 or x2.dim() != 2 or \
            xq.shape[1] != x2.shape[1] or xq.shape[0] < x2.shape[0]:
        return
    if torch.compiler.is_compiling():
        (_OP[0] if _OP[0] is not None else quant_op())(x2, xq, xs, recipe, scale_ub, static_ref, rows_buf, stepbuf,
                                                       state, slot, int(mult))
    else:
        quant_check(x2, xq, xs, recipe, scale_ub, static_ref, rows_buf, stepbuf, state, slot, int(mult))


def _per_tensor(gs) -> bool:
    """Whether a quantizer's group shape is per tensor: a (row, col) pair of -1s, an is_per_tensor() method, or a
    name containing TENSOR."""
    f = getattr(gs, "is_per_tensor", None)
    if callable(f):
        try:
            return bool(f())
        except Exception:  # noqa: BLE001
            return False
    if isinstance(gs, tuple) and len(gs) == 2:
        return tuple(gs) == (-1, -1)
    return "TENSOR" in str(getattr(gs, "name", gs) or "").upper()


def recipe_of(quant_fp8) -> tuple:
    """(recipe, why not) of a layer's FP8 input quantizer (serve_fp8.py:236-248)."""
    if quant_fp8 is None:
        return None, "no FP8 input quantization found"
    if getattr(quant_fp8, "is_group_quant", False):
        return None, "FP8 with group (block) activation scales"
    gs = getattr(quant_fp8, "group_shape", None)
    if getattr(quant_fp8, "static", False):
        if not _per_tensor(gs):
            return None, f"static FP8 activation scales per {getattr(gs, 'name', gs) or 'group'}"
        return RECIPES["static"], None
    if getattr(quant_fp8, "use_per_token_if_dynamic", False):
        return RECIPES["dynamic_token"], None
    return RECIPES["dynamic_tensor"], None


_FINDINGS = {KIND_OUTSIDE: "scale_from_outside_rows", KIND_SCALE: "scale_wrong", KIND_VALUES: "values_wrong",
             KIND_STATIC: "static_scale_changed"}
_READING = {
    "scale_from_outside_rows": "the per-tensor FP8 scale the GEMM used is the maximum over every row of its input, "
                               "padding included, not over this step's real rows: the output depends on rows an "
                               "earlier request left",
    "scale_wrong": "the FP8 scale the GEMM used differs from the scale its recipe gives for this step's rows",
    "values_wrong": "FP8 values the GEMM got are two or more FP8 steps from the layer's input quantized with that "
                    "scale",
    "static_scale_changed": "the layer's static FP8 input scale changed since load",
}


class Fp8Checks:
    """The FP8 layers whose quantization one serving guard checks: add() each at weight processing, mark_step(step,
    rows) before each model step and end_step() after it, poll() to read the counters (serve_fp8.py:251-419)."""

    def __init__(self, guard=None):
        self._marked: Optional[int] = None
        self.guard = guard
        self.layers: list = []
        self.unsupported: dict = {}
        self._state, self._rows, self._step, self._host = {}, {}, {}, {}
        self.stats = {"layers": 0, "calls": 0, "scale_wrong": 0, "scale_from_outside_rows": 0, "values_wrong": 0,
                      "fp8_one_step": 0, "alerts": 0}
        self.seen: dict = {}
        self.events: list = []
        self._lock = threading.Lock()

    def _dev(self, dev):
        if dev not in self._state:
            with torch.inference_mode(False):
                self._state[dev] = torch.zeros(64, COLS, dtype=torch.int64, device=dev)
                self._rows[dev] = torch.zeros(1, dtype=torch.int64, device=dev)
                self._step[dev] = torch.zeros(1, dtype=torch.int64, device=dev)
        return self._state[dev]

    def add(self, layer, name: str, quant_fp8, static_scale: Optional[torch.Tensor], device) -> Optional[tuple]:
        """Register one layer; its call arguments (for check_call), or None with the reason in unsupported."""
        device = torch.device(device)
        recipe, why = recipe_of(quant_fp8)
        if why:
            self.unsupported[name] = why
            return None
        if device.type != "cuda":
            self.unsupported[name] = "not on a GPU"
            return None
        with self._lock:
            st = self._dev(device)
            slot = sum(1 for lay in self.layers if lay["device"] == device)
            if slot >= st.shape[0]:
                with torch.inference_mode(False):
                    grown = torch.zeros(st.shape[0] * 2, COLS, dtype=torch.int64, device=device)
                    grown[:st.shape[0]] = st
                self._state[device] = grown
                for lay in self.layers:               # their arguments hold the old rows: point them at the new ones
                    if lay["device"] == device and lay["layer"] is not None:
                        lay["layer"]._sdcguard_fp8 = self.args(lay)
            ref = None
            if recipe == RECIPES["static"] and isinstance(static_scale, torch.Tensor):
                with torch.inference_mode(False):
                    ref = static_scale.detach().float().reshape(-1)[:1].clone()
            lay = {"name": name, "layer": layer, "device": device, "slot": slot, "recipe": recipe, "static_ref": ref}
            self.layers.append(lay)
            self.stats["layers"] += 1
            quant_op()
            a = self.args(lay)
            if layer is not None:
                layer._sdcguard_fp8 = a
            return a

    def args(self, lay) -> tuple:
        dev = lay["device"]
        return (lay["recipe"], lay["static_ref"], self._rows[dev], self._step[dev], self._state[dev], lay["slot"])

    def mark_step(self, step: int, rows: Optional[int] = None) -> None:
        """Publish the coming step and its real row count on every device (fills: no host synchronisation)."""
        self._marked = int(step) & M32
        for dev in self._state:
            self._step[dev].fill_(int(step) & M32)
            self._rows[dev].fill_(int(rows) if rows is not None else 0)

    def end_step(self) -> None:
        for dev in self._state:
            self._rows[dev].zero_()

    def detach(self) -> None:
        try:
            self.poll(wait=True)
        finally:
            for lay in self.layers:
                if lay["layer"] is not None:
                    lay["layer"].__dict__.pop("_sdcguard_fp8", None)
                    lay["layer"].__dict__.pop("_sdcguard_fp8_moe", None)
            self.layers.clear()
            for d in (self._state, self._rows, self._step, self._host):
                d.clear()

    def coverage(self) -> dict:
        return {"layers": len(self.layers), "calls": self.stats["calls"],
                "layers_checked": sum(self.seen.get(lay["name"], 0) > 0 for lay in self.layers),
                "never_checked": sorted(lay["name"] for lay in self.layers if not self.seen.get(lay["name"])),
                "not_attached": dict(self.unsupported), "samples_per_call": SAMPLES,
                "recipes": sorted({k for lay in self.layers for k, v in RECIPES.items() if v == lay["recipe"]})}

    def poll(self, wait: bool = False) -> list:
        """Counters read back and cleared.  Without wait the copy is started now and reported by a later poll."""
        events = []
        for dev, st in list(self._state.items()):
            if wait:
                pend = self._host.pop(dev, None)
                if pend is not None:
                    pend[1].synchronize()
                    events += self._report(dev, pend[0])
                host = st.to("cpu", copy=True)
                st.zero_()
                events += self._report(dev, host)
                continue
            pend = self._host.get(dev)
            if pend is not None and pend[1].query():
                events += self._report(dev, pend[0])
                self._host.pop(dev, None)
                pend = None
            if pend is None:
                hs = torch.empty(st.shape, dtype=st.dtype, pin_memory=True)
                hs.copy_(st, non_blocking=True)
                st.zero_()
                ev = torch.cuda.Event()
                ev.record(torch.cuda.current_stream(dev))
                self._host[dev] = (hs, ev)
        return events

    def _report(self, dev, host) -> list:
        out = []
        for lay in self.layers:
            if lay["device"] != dev or lay["slot"] >= host.shape[0]:
                continue
            k = [int(v) for v in host[lay["slot"]].tolist()]
            self.stats["calls"] += k[C_CALLS]
            self.seen[lay["name"]] = self.seen.get(lay["name"], 0) + k[C_CALLS]
            self.stats["scale_wrong"] += k[C_SCALE]
            self.stats["scale_from_outside_rows"] += k[C_OUTSIDE]
            self.stats["values_wrong"] += k[C_VALUES]
            self.stats["fp8_one_step"] += k[C_ONE]
            if k[C_SCALE] or k[C_VALUES] or k[C_STATIC]:
                out.append(self._alert(lay, k))
        return out

    def _alert(self, lay, k) -> SDCEvent:
        last = k[C_LAST]
        step, kind, row = unwrap31(last >> 32, self._marked), (last >> 24) & 0xFF, last & 0xFFFFFF
        what = _FINDINGS.get(kind, "unknown")
        detail = {"where": lay["name"], "kind": "fp8_quantization", "finding": what, "calls_judged": k[C_CALLS],
                  "calls_with_wrong_scale": k[C_SCALE], "calls_scale_from_outside_rows": k[C_OUTSIDE],
                  "sampled_rows_with_wrong_values": k[C_VALUES], "values_one_fp8_step_off": k[C_ONE],
                  "scale_ratio": _f32(k[C_RATIO]) if k[C_RATIO] else None,
                  "captured": ({"step": step, "row": None, "every_row": True} if row == EVERY_ROW else
                               {"step": step, "row": row}) if kind in (KIND_VALUES, KIND_SCALE, KIND_OUTSIDE) else None,
                  "recipe": next(n for n, v in RECIPES.items() if v == lay["recipe"]),
                  "check_config": {"samples_per_call": SAMPLES, "scale_tolerance": SCALE_TOL,
                                   "values": "2 or more FP8 steps off is an alarm; 1 step is counted (fast math)"},
                  "reading": _READING.get(what, "")}
        ev = SDCEvent(detector="serve_fp8", layer=lay["name"], z=float("inf"), row=None if row == EVERY_ROW else row,
                      extra=detail)
        self.stats["alerts"] += 1
        self.events.append(ev)
        g = self.guard
        if g is not None and getattr(g, "on_alert", None):
            try:
                g.on_alert(ev)
            except Exception:  # noqa: BLE001  (an alert callback never breaks serving)
                pass
        return ev
