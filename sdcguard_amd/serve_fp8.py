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

import threading
from typing import Optional

import torch

from .stepchecks import W_ROWS, W_STEP, Binding, Registered, StepChecks, f32_of

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

_OP_LOCK = threading.Lock()
_OP: list = [None]


def quant_op():
    """The check as one opaque op for torch.compile, registered on first use under the reference's name and schema
    (sdcguard::fp8_quant_check, serve_fp8.py:181-205); where the op cannot be registered, the library call."""
    with _OP_LOCK:
        if _OP[0] is not None:
            return _OP[0]
        op = getattr(getattr(torch.ops, "sdcguard", None), "fp8_quant_check", None)
        if op is None:
            try:
                lib_op = torch.library.custom_op("sdcguard::fp8_quant_check", mutates_args=("state",))(_op_body)
                lib_op.register_fake(lambda *a: None)
                op = torch.ops.sdcguard.fp8_quant_check
            except (AttributeError, RuntimeError):
                op = quant_check
        _OP[0] = op
        return op


def _op_body(x2: torch.Tensor, xq: torch.Tensor, xs: torch.Tensor, recipe: int, scale_ub: Optional[torch.Tensor],
             static_ref: Optional[torch.Tensor], rows_buf: torch.Tensor, stepbuf: torch.Tensor, state: torch.Tensor,
             slot: int, mult: int) -> None:
    quant_check(x2, xq, xs, recipe, scale_ub, static_ref, rows_buf, stepbuf, state, slot, mult)


def _shapes_fit(x2, xq, xs) -> bool:
    return isinstance(xq, torch.Tensor) and isinstance(xs, torch.Tensor) and x2.dim() == 2 and xq.dim() == 2 and \
        xq.shape[1] == x2.shape[1] and xq.shape[0] >= x2.shape[0]


def check_call(binding, x2: torch.Tensor, xq: torch.Tensor, xs: torch.Tensor,
               scale_ub: Optional[torch.Tensor] = None, mult: int = 1) -> None:
    """One quantization of a registered layer (its input, the FP8 input its GEMM got and that input's scale), queued
    on the current stream.  binding: what Fp8Checks.add returned (serve_fp8.py:208-219)."""
    if binding is None or not _shapes_fit(x2, xq, xs):
        return
    args = binding.checks.call_args(binding)
    run = quant_op() if torch.compiler.is_compiling() else quant_check
    run(x2, xq, xs, args[0], scale_ub, args[1], args[2], args[3], args[4], args[5], max(int(mult), 1))


# How a quantizer object of the serving stack tells its recipe (serve_fp8.py:236-248 reads the same attributes):
# group (block) scales are not checked; a static scale must be one for the whole tensor; a dynamic one is per token
# when the quantizer says so, else per tensor.
def _is_whole_tensor(group_shape) -> bool:
    probe = getattr(group_shape, "is_per_tensor", None)
    if callable(probe):
        try:
            return bool(probe())
        except Exception:  # noqa: BLE001
            return False
    if isinstance(group_shape, tuple):
        return len(group_shape) == 2 and all(int(v) == -1 for v in group_shape)
    label = getattr(group_shape, "name", group_shape)
    return label is not None and "TENSOR" in str(label).upper()


def recipe_of(quant_fp8) -> tuple:
    """(recipe code, None) of an FP8 input quantizer, or (None, why it is not checked)."""
    if quant_fp8 is None:
        return None, "no FP8 input quantization found"
    if bool(getattr(quant_fp8, "is_group_quant", False)):
        return None, "FP8 with group (block) activation scales"
    if not bool(getattr(quant_fp8, "static", False)):
        token = bool(getattr(quant_fp8, "use_per_token_if_dynamic", False))
        return RECIPES["dynamic_token" if token else "dynamic_tensor"], None
    gs = getattr(quant_fp8, "group_shape", None)
    if _is_whole_tensor(gs):
        return RECIPES["static"], None
    return None, f"static FP8 activation scales per {getattr(gs, 'name', gs) or 'group'}"


_FINDINGS = {KIND_OUTSIDE: "scale_from_outside_rows", KIND_SCALE: "scale_wrong", KIND_VALUES: "values_wrong",
             KIND_STATIC: "static_scale_changed"}
_MEANING = {
    "scale_from_outside_rows": "the GEMM's per-tensor scale is the largest |x| over all its input rows, padding "
                               "included; over this step's own rows it is smaller, so the result depended on rows "
                               "left by an earlier request",
    "scale_wrong": "the GEMM's FP8 scale is not the one its recipe gives for this step's rows",
    "values_wrong": "sampled FP8 inputs of the GEMM are two or more E4M3 steps from the layer's input quantized with "
                    "the GEMM's scale",
    "static_scale_changed": "the layer's static FP8 input scale is not its value at load",
}


class Fp8Checks(StepChecks):
    """FP8 input quantizations checked for one serving guard.  add() each FP8 layer at load (it returns the binding
    the layer's call site passes to check_call); mark_step / end_step around each model step; poll() to read.
    State rows are the kernel's 8 counters per layer (the reference's columns, serve_fp8.py:46-50)."""

    DETECTOR = "serve_fp8"
    COLS = COLS

    def __init__(self, guard=None):
        super().__init__(guard)
        self.stats.update(calls=0, scale_wrong=0, scale_from_outside_rows=0, values_wrong=0, fp8_one_step=0)
        self.seen: dict = {}

    def add(self, layer, name: str, quant_fp8, static_scale: Optional[torch.Tensor], device) -> Optional[Binding]:
        recipe, why = recipe_of(quant_fp8)
        if why is None and torch.device(device).type != "cuda":
            why = "not on a GPU"
        if why:
            self._refuse(name, why)
            return None
        ref = None
        if recipe == RECIPES["static"] and isinstance(static_scale, torch.Tensor):
            with torch.inference_mode(False):
                ref = static_scale.detach().float().reshape(-1)[:1].clone()
        b = self._register(name, layer, device, recipe=recipe, static_ref=ref)
        quant_op()
        if layer is not None:
            layer._sdcguard_fp8 = b
        return b

    def call_args(self, b: Binding) -> tuple:
        """(recipe, static reference, real rows, step, state, slot) of a binding's layer, as the kernel takes them."""
        lay, tab = b.layer, b.table()
        return (lay.info["recipe"], lay.info["static_ref"], tab.word.view(W_ROWS), tab.word.view(W_STEP), tab.state,
                lay.slot)

    def _unbind(self, lay: Registered) -> None:
        if lay.module is not None:
            for attr in ("_sdcguard_fp8", "_sdcguard_fp8_moe"):
                lay.module.__dict__.pop(attr, None)

    def coverage(self) -> dict:
        out = super().coverage()
        out.update(calls=self.stats["calls"], samples_per_call=SAMPLES,
                   recipes=sorted({n for n, v in RECIPES.items() for lay in self.layers if lay.info["recipe"] == v}))
        return out

    def _count(self, lay: Registered, k: list) -> None:
        lay.calls += k[C_CALLS]
        self.seen[lay.name] = self.seen.get(lay.name, 0) + k[C_CALLS]
        for stat, col in (("calls", C_CALLS), ("scale_wrong", C_SCALE), ("scale_from_outside_rows", C_OUTSIDE),
                          ("values_wrong", C_VALUES), ("fp8_one_step", C_ONE)):
            self.stats[stat] += k[col]

    def _judged(self, k: list) -> bool:
        return k[C_CALLS] > 0

    def _judge(self, lay: Registered, k: list, captured: dict, window) -> list:
        if not (k[C_SCALE] or k[C_VALUES] or k[C_STATIC]):
            return []
        step = unwrap31(k[C_LAST] >> 32, self.marked)
        kind, row = (k[C_LAST] >> 24) & 0xFF, k[C_LAST] & 0xFFFFFF
        finding = _FINDINGS.get(kind, "unknown")
        where = None
        if kind in (KIND_VALUES, KIND_SCALE, KIND_OUTSIDE):
            where = {"step": step, "row": None, "every_row": True} if row == EVERY_ROW else {"step": step, "row": row}
        recipe = next(n for n, v in RECIPES.items() if v == lay.info["recipe"])
        detail = {"where": lay.name, "kind": "fp8_quantization", "finding": finding, "recipe": recipe,
                  "calls_judged": k[C_CALLS], "calls_with_wrong_scale": k[C_SCALE],
                  "calls_scale_from_outside_rows": k[C_OUTSIDE], "sampled_rows_with_wrong_values": k[C_VALUES],
                  "values_one_fp8_step_off": k[C_ONE], "scale_ratio": f32_of(k[C_RATIO]) if k[C_RATIO] else None,
                  "captured": where, "read_window_steps": window, "last_clean_read_steps": self.last_clean(lay.name),
                  "check_config": {"samples_per_call": SAMPLES, "scale_tolerance": SCALE_TOL,
                                   "values": "an alarm from 2 E4M3 steps off; 1 step is counted only"},
                  "reading": _MEANING.get(finding, "")}
        return [self.emit(lay, float("inf"), None if row == EVERY_ROW else row, detail)]
