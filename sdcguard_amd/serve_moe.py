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
import threading
from typing import Optional

import torch

from .stepchecks import W_PACKED, Binding, Registered, StepChecks, f32_of, pack_step

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

_OP_LOCK = threading.Lock()
_OP: list = [None]


def moe_op():
    """The check as one opaque op for torch.compile, registered once under the reference's name (sdcguard::moe_check);
    where the op cannot be registered, the library call."""
    with _OP_LOCK:
        if _OP[0] is not None:
            return _OP[0]
        op = getattr(getattr(torch.ops, "sdcguard", None), "moe_check", None)
        if op is None:
            try:
                lib_op = torch.library.custom_op(
                    "sdcguard::moe_check", mutates_args=("state", "cap_meta", "cap_x", "cap_y", "cap_ids", "cap_g"))(
                        _op_body)
                lib_op.register_fake(lambda *a: None)
                op = torch.ops.sdcguard.moe_check
            except (AttributeError, RuntimeError):
                op = moe_check
        _OP[0] = op
        return op


def _op_body(x: torch.Tensor, out: torch.Tensor, topk_w: torch.Tensor, topk_ids: torch.Tensor, w13: torch.Tensor,
             w2: torch.Tensor, expert_map: Optional[torch.Tensor], act: int, routed_first: bool, state: torch.Tensor,
             slot: int, stepbuf: torch.Tensor, nlayers: int, index: int, cap_meta: torch.Tensor, cap_x: torch.Tensor,
             cap_y: torch.Tensor, cap_ids: torch.Tensor, cap_g: torch.Tensor, line: float) -> None:
    moe_check(x, out, topk_w, topk_ids, w13, w2, expert_map, act, routed_first, state, slot, stepbuf, nlayers, index,
              cap_meta, cap_x, cap_y, cap_ids, cap_g, line)


def check_call(binding, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor, out) -> None:
    """After one call of a registered MoE layer: its input, routing and (finalized) output.  binding: the layer's
    _sdcguard_moe (set by MoEChecks.finalize)."""
    if binding is None or not (isinstance(out, torch.Tensor) and isinstance(x, torch.Tensor)):
        return
    if out.shape[-1] != x.shape[-1] or out.shape[0] != x.shape[0]:
        return
    args = binding.checks.call_args(binding)
    if torch.compiler.is_compiling():
        moe_op()(x, out, topk_weights, topk_ids, *args)
        return
    with torch.no_grad():
        moe_check(x, out, topk_weights, topk_ids, *args)


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
    worst = f32_of(keys[C_ROW] >> 32)
    bad = int((z > line).sum())
    out = {"worst_score": worst, "outputs_over_line": bad, "outputs": h, "experts": used}
    if worst > 0:
        out.update(col=keys[C_COL] & M32, output=f32_of(keys[C_OUT]), expected=f32_of(keys[C_REF]))
    if bad:
        return {**out, "verdict": "output_wrong",
                "why": f"{bad} of {h} outputs of the kept row are farther from the recompute (the layer's current "
                       "weights, the kept input and routing) than its rounding allows"}
    return {**out, "verdict": "output_agrees",
            "why": "the recompute of the kept row alone agrees with its output: the check disagreed when the row "
                   "ran in its batch, or the weights changed back since"}


# ------------------------------------------------------------------------------------------------- the MoE layers
def _across_gpus(mod) -> bool:
    """Whether the layer's rows or outputs combine other GPUs' (all-to-all, data or prefill-context parallelism)."""
    pc = getattr(getattr(mod, "moe_config", None), "moe_parallel_config", None)
    try:
        flags = [getattr(pc, f, False) for f in ("use_all2all_kernels", "use_passthrough_all2all")]
        sizes = [int(getattr(pc, f, 1) or 1) for f in ("dp_size", "pcp_size")]
    except Exception:  # noqa: BLE001  (an unreadable config counts as combined)
        return True
    return any(bool(f) for f in flags) or any(v > 1 for v in sizes)


def _experts(mod):
    w13, w2 = getattr(mod, "w13_weight", None), getattr(mod, "w2_weight", None)
    ok = isinstance(w13, torch.Tensor) and isinstance(w2, torch.Tensor) and w13.dim() == 3 and w2.dim() == 3
    return (w13, w2) if ok else (None, None)


def _activation(mod) -> str:
    a = getattr(mod, "activation", None)
    return str(getattr(a, "value", a))


# What a fused MoE layer must be for the recompute to model it (the reference's serve_moe.py:709-748 asks the same
# of the serving stack's layer): each rule is (holds, why not), tried in order.
_RULES = (
    (lambda m: type(getattr(m, "quant_method", None)).__name__ == "UnquantizedFusedMoEMethod",
     lambda m: f"{type(getattr(m, 'quant_method', None)).__name__}: quantized or another method"),
    (lambda m: not _across_gpus(m),
     lambda m: "expert parallelism's all-to-all, data parallelism or prefill context parallelism: the layer's rows or "
               "output combine other GPUs'"),
    (lambda m: getattr(getattr(m.quant_method, "unquantized_backend", None), "name", None) == "TRITON",
     lambda m: f"the {getattr(getattr(m.quant_method, 'unquantized_backend', None), 'name', None) or 'unknown'} MoE "
               "backend (the recompute models the Triton MoE kernel's roundings)"),
    (lambda m: _experts(m)[0] is not None, lambda m: "no expert weights the check knows"),
    (lambda m: _experts(m)[0].dtype in (torch.bfloat16, torch.float16) and _experts(m)[1].dtype == _experts(m)[0].dtype,
     lambda m: f"expert weights in {_experts(m)[0].dtype}"),
    (lambda m: _experts(m)[0].shape[0] == _experts(m)[1].shape[0] and _experts(m)[0].shape[2] == _experts(m)[1].shape[1]
     and _experts(m)[0].shape[1] == 2 * _experts(m)[1].shape[2],
     lambda m: f"expert weight shapes {tuple(_experts(m)[0].shape)} and {tuple(_experts(m)[1].shape)} aren't gate-up "
               "and down"),
    (lambda m: _experts(m)[0].shape[2] <= 8192, lambda m: f"hidden size {_experts(m)[0].shape[2]} (at most 8192)"),
    (lambda m: not any(isinstance(getattr(m, b, None), torch.Tensor) for b in ("w13_bias", "w2_bias")),
     lambda m: "experts with biases"),
    (lambda m: _activation(m) in ACT, lambda m: f"activation {_activation(m)}"),
    (lambda m: _experts(m)[0].is_cuda, lambda m: "not on a GPU"),
    (lambda m: getattr(m, "_sdcguard_moe", None) is None, lambda m: "already checked by another ServeGuard"),
)


def describe(mod) -> tuple:
    """(what the check needs of a fused MoE layer, None), or (None, why it is not checked)."""
    for holds, why in _RULES:
        if not holds(mod):
            return None, why(mod)
    return {"act": ACT[_activation(mod)], "routed_first": bool(getattr(mod, "apply_router_weight_on_input", False)),
            "top_k": int(getattr(mod, "top_k", 0) or 0)}, None


def _weights_id(mod) -> torch.Tensor:
    """The experts' weights as two exact integer fingerprints each (sdc_fingerprint2), on their device."""
    from .serve_weights import fingerprint
    return torch.stack([fingerprint(mod.w13_weight.detach()), fingerprint(mod.w2_weight.detach())])


_ROUTE_WHY = ("a real token's row came with expert ids of -1 or out of range (every real token gets top_k experts; "
              "-1 marks padding rows), so the layer's output for it is not the sum of its experts")


class MoEChecks(StepChecks):
    """The fused MoE layers one serving guard checks: add() each, finalize() once before any graph is captured (it
    numbers the layers' turns: at step s the layer with index s % layers recomputes), mark_step() / end_step() around
    each model step, poll() to read.  State rows are the kernel's 11 columns (the reference's, serve_moe.py:60-70)."""

    DETECTOR = "serve_moe"
    COLS = COLS
    CAPTURE = {"meta": torch.int32, "x": torch.float32, "y": torch.float32, "ids": torch.int64, "g": torch.float32}
    READ_CAPTURE = ("meta",)

    def __init__(self, guard=None, line: float = MOE_Z):
        line = float(line)
        if not 5.0 <= line < float("inf"):
            raise ValueError(f"the MoE check's line must be at least 5, not {line!r}")
        super().__init__(guard)
        self.line = line
        self.finalized = False
        self.worst_seen: dict = {}
        self.checks_seen: dict = {}
        self.stats.update(active_calls=0, rows_checked=0, unjudged_outputs=0, unrouted_real_rows=0,
                          partly_routed_real_rows=0)

    def add(self, mod, name: str) -> Optional[int]:
        if self.finalized:
            raise RuntimeError("MoE layers are added before finalize()")
        info, why = describe(mod)
        if why:
            self._refuse(name, why)
            return None
        h, k = int(mod.w13_weight.shape[2]), max(info["top_k"], 1)
        with torch.inference_mode(False), torch.no_grad():
            ident = _weights_id(mod)
        b = self._register(name, mod, mod.w13_weight.device,
                           widths={"meta": CAP_COLS, "x": h, "y": h, "ids": max(k, 64), "g": max(k, 64)},
                           h=h, i=int(mod.w2_weight.shape[2]), k=k, ident=ident, **info)
        return b.slot

    def finalize(self) -> int:
        """Number each device's layers' turns, reserve the kernels' workspace, register the op and give each layer
        its binding (before any graph is captured: the tables' addresses are fixed from here on)."""
        if self.finalized:
            return len(self.layers)
        from . import _lib
        per_dev: dict = {}
        for lay in self.layers:
            per_dev.setdefault(lay.device, []).append(lay)
        for dev, lays in per_dev.items():
            for turn, lay in enumerate(lays):
                lay.info["index"], lay.info["nlayers"] = turn, len(lays)
            _lib.workspace(dev, max(int(_lib.lib().sdc_moe_check_workspace(lay.info["h"], lay.info["i"],
                                                                            lay.info["k"])) for lay in lays))
        moe_op()
        for n, lay in enumerate(self.layers):
            lay.module._sdcguard_moe = Binding(self, n)
        self.finalized = True
        return len(self.layers)

    def call_args(self, b: Binding) -> tuple:
        """The library call's arguments after (x, out, topk_w, topk_ids) for a binding's layer."""
        lay, tab = b.layer, b.table()
        c = tab.capture
        return (lay.module.w13_weight, lay.module.w2_weight, getattr(lay.module, "expert_map", None),
                lay.info["act"], lay.info["routed_first"], tab.state, lay.slot, tab.word.view(W_PACKED),
                lay.info["nlayers"], lay.info["index"], c["meta"], c["x"], c["y"], c["ids"], c["g"], self.line)

    def args(self, slot: int) -> tuple:
        return self.call_args(Binding(self, slot))

    def refresh(self) -> int:
        """Take the experts' current weights as their own (after an intended update)."""
        with torch.inference_mode(False), torch.no_grad():
            for lay in self.layers:
                lay.info["ident"] = _weights_id(lay.module)
                lay.info.pop("restored", None)
        return len(self.layers)

    def weights_restored(self, module, step) -> None:
        """The weight scan's repair wrote these experts' load-time weights back after `step`."""
        for lay in self.layers:
            if lay.module is module:
                lay.info["restored"] = {"step": step}

    def detach(self) -> None:
        super().detach()
        self.finalized = False

    def _unbind(self, lay: Registered) -> None:
        lay.module.__dict__.pop("_sdcguard_moe", None)

    def coverage(self) -> dict:
        out = super().coverage()
        out.update(active_calls=self.stats["active_calls"], samples_per_step=SAMPLES)
        return out

    def _count(self, lay: Registered, k: list) -> None:
        lay.calls += k[C_CALLS]
        self.checks_seen[lay.name] = self.checks_seen.get(lay.name, 0) + k[C_CALLS]
        for stat, col in (("active_calls", C_CALLS), ("rows_checked", C_ROWS), ("unjudged_outputs", C_UNJ),
                          ("unrouted_real_rows", C_UNROUTED), ("partly_routed_real_rows", C_PARTIAL)):
            self.stats[stat] += k[col]

    def _judged(self, k: list) -> bool:
        return k[C_CALLS] > 0 and not (k[C_UNROUTED] or k[C_PARTIAL])

    def _judge(self, lay: Registered, k: list, captured: dict, window) -> list:
        out = []
        if k[C_UNROUTED] or k[C_PARTIAL]:
            out.append(self._routing_event(lay, k, window))
        z = f32_of(k[C_ROW] >> 32)
        self.worst_seen[lay.name] = max(self.worst_seen.get(lay.name, 0.0), z)
        lay.worst = max(lay.worst, z)
        if z > self.line:
            meta = [int(v) for v in captured["meta"].tolist()] if "meta" in captured else [0, 0, 0, 0]
            out.append(self._output_event(lay, k, meta, window, z))
        return out

    def _routing_event(self, lay: Registered, k: list, window) -> object:
        row = (k[C_BADROW] & M32) - 1
        step = (k[C_BADROW] >> 32) & M32
        detail = {"where": lay.name, "kind": "moe_routing",
                  "finding": "real_rows_unrouted" if k[C_UNROUTED] else "real_rows_partly_routed",
                  "real_rows_without_experts": k[C_UNROUTED], "real_rows_missing_some_experts": k[C_PARTIAL],
                  "row": row if row >= 0 else None,
                  "captured": {"row": row, "step": step if self.marked is not None else None} if row >= 0 else None,
                  "recheck": {"verdict": "output_wrong", "why": _ROUTE_WHY},
                  "read_window_steps": window, "last_clean_read_steps": self.last_clean(lay.name),
                  "reading": "a real row reached the experts without (some of) its experts: a router fault, a "
                             "corrupted expert id, or a padding mask over a real row"}
        return self.emit(lay, math.inf, detail["row"], detail)

    def _kept_row(self, lay: Registered, meta: list) -> tuple:
        """The kept row's record (input, output, experts, weights), read from the device, and its capture freed."""
        if not meta[0]:
            return None, None
        c = self.tables[lay.device].capture
        h, k = lay.info["h"], lay.info["k"]
        rec = (c["x"][lay.slot, :h].clone(), c["y"][lay.slot, :h].clone(), c["ids"][lay.slot, :k].clone(),
               c["g"][lay.slot, :k].clone())
        c["meta"][lay.slot].zero_()
        kept = {"row": meta[1] & M32, "step": (meta[2] & M32) if self.marked is not None else None,
                "score": f32_of(meta[3]), "experts": rec[2].tolist(), "weights": rec[3].tolist()}
        return kept, rec

    def _output_event(self, lay: Registered, k: list, meta: list, window, z: float) -> object:
        mod = lay.module
        dtype = mod.w13_weight.dtype
        kept, rec = self._kept_row(lay, meta)
        verdict = None
        if rec is not None:
            try:
                verdict = recheck(rec[0], rec[1], rec[2].to(torch.int32), rec[3], mod.w13_weight, mod.w2_weight,
                                  getattr(mod, "expert_map", None), lay.info["act"], lay.info["routed_first"], dtype,
                                  self.line)
            except Exception as e:  # noqa: BLE001  (the diagnosis is best effort)
                verdict = {"verdict": "not_rechecked", "why": f"{type(e).__name__}: {e}"}
        try:
            with torch.no_grad():
                changed = not torch.equal(_weights_id(mod).cpu(), lay.info["ident"].cpu())
        except Exception:  # noqa: BLE001
            changed = None
        if verdict is not None and changed and verdict.get("verdict") == "output_agrees":
            verdict = {**verdict, "verdict": "weights_changed",
                       "why": "the kept row agrees with a recompute from the experts' weights as they are now, and "
                              "those differ from the weights at load: the weights changed in memory (refresh() after "
                              "an intended update)"}
        if verdict is not None and kept is not None:
            from .serve_weights import before_repair, repair_why
            if before_repair(lay.info.get("restored"), kept["step"]):
                verdict = {**verdict, "verdict": "unknown", "why": repair_why(lay.info["restored"], kept["step"])}
        row, col, yv, rv, place = k[C_ROW] & M32, k[C_COL] & M32, f32_of(k[C_OUT]), f32_of(k[C_REF]), PLACE_MAXIMA
        if kept is not None and verdict and verdict.get("outputs_over_line") and verdict.get("col") is not None:
            row, col, yv, rv, place = kept["row"], verdict["col"], verdict["output"], verdict["expected"], PLACE_KEPT
        detail = {"where": lay.name, "kind": "moe_experts", "max_z": z, "row": row, "col": col, "output": yv,
                  "expected": rv, "place": place,
                  "relative_error": abs(yv - rv) / abs(rv) if rv and rv == rv else None, "captured": kept,
                  "recheck": verdict or {"verdict": "not_rechecked",
                                         "why": "no row was kept for this alert (an earlier alert's kept row has not "
                                                "been read yet)"},
                  "weights_changed_since_load": changed, "read_window_steps": window,
                  "last_clean_read_steps": self.last_clean(lay.name),
                  "check_config": {"line": self.line, "samples_per_step": SAMPLES, "kappa": KAPPA, "flips": FLIPS,
                                   "unit_roundoff": dtype_consts(dtype)[0],
                                   "reference": "sampled recompute with the fused MoE kernel's rounding steps"},
                  "reading": "an output of the layer's routed experts is farther from a recompute from the layer's "
                             "own input, routing and weights than the kernel's roundings allow"}
        return self.emit(lay, z, row, detail)
