"""Checks of MoE routing in serving: did a router pick the experts and weights its routing policy gives for its
logits?  (reference: serve_route.py)

A fused MoE layer's router turns each token's logits into its top-k experts and their weights by the model's policy:
softmax or sigmoid scores; a correction bias added for choosing, not for the weights; DeepSeek's grouped top-k (the
best topk_group groups first, a group scored by its two best biased scores, or its best score without a bias); the
weights renormalized over the chosen experts or not, then scaled.  A wrong expert is an output from the wrong
weights with nothing wrong in the experts' arithmetic, so the experts' recompute (serve_moe) cannot see it.

At each model step one router (index = step modulo the routers on its GPU) recomputes its policy in fp32 for
SAMPLES real rows of the step and judges the router's result: each chosen expert's choice score at least the k-th
best the policy allows, less a tie tolerance (1e-6 of the size, plus 4 unit roundoffs of 16-bit logits; groups near
the cut within twice that may go either way), the k ids distinct; the weights to 2e-5 + (1e-4 + 6u) of their size.
A row of all -1 ids is padding and isn't judged.

The arithmetic is one launch of the HIP library (route_check.hip, sdc_route_check) that returns at once for the
routers not on turn: no host synchronisation, no memory set, so it is captured with the step in a graph.  The host
side here is:
  route_check     one call, with the reference's operator arguments (route_check_torch, :141-184)
  route_op        the same as one opaque op (sdcguard::route_check) for torch.compile
  policy_of       which vLLM routers the check models, and their policy (the reference's rules, :552-585)
  RouteChecks     the routers one ServeGuard checks, on the shared per-step machinery of stepchecks.py
Not checked (listed by RouteChecks.unsupported): custom routing functions, hash routing, image-token biases, fused
shared experts, expert load balancing (physical expert ids), and kernels that route inside the MoE kernel.
"""
from __future__ import annotations

import math
import threading
from typing import Optional

import torch

from .stepchecks import W_ROWS, W_STEP, Binding, Registered, StepChecks, f32_of

SAMPLES = 2
COLS = 6
# state row: calls judged, rows with a wrong expert set, rows with a wrong weight, last wrong row
# ((step & S31) << 32 | kind << 24 | row), worst weight difference (float bits), rows judged
C_CALLS, C_SET, C_WEIGHT, C_LAST, C_WDIFF, C_ROWS = range(COLS)
KIND_SET, KIND_WEIGHT = 2, 1
CAP_COLS = 6                     # kept row: taken, row, step, kind, experts, logits dtype code
MAX_EXPERTS, MAX_K, MAX_GROUPS = 2048, 32, 64
SCORING = {"softmax": 0, "sigmoid": 1}
DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
CODE_DTYPE = {v: k for k, v in DTYPE_CODE.items()}
_WEIGHT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
_ID_CODE = {torch.int32: 0, torch.int64: 1}
S31 = 0x7FFFFFFF
M32 = 0xFFFFFFFF


def unit_roundoff(dtype: torch.dtype) -> float:
    """Half the epsilon of 16-bit logits; 0 for fp32 (the 1e-6 tie covers it)."""
    return float(torch.finfo(dtype).eps) / 2 if dtype in (torch.bfloat16, torch.float16) else 0.0


def _last_dense(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def route_check(logits: torch.Tensor, topk_w: torch.Tensor, topk_ids: torch.Tensor, k: int, scoring: int,
                renormalize: bool, bias: Optional[torch.Tensor], groups: int, topk_group: int, scale: float,
                rows_buf: torch.Tensor, stepbuf: torch.Tensor, state: torch.Tensor, slot: int, nlayers: int,
                index: int, cap_meta: torch.Tensor, cap_lg: torch.Tensor, cap_ids: torch.Tensor,
                cap_w: torch.Tensor) -> None:
    """One router call's check queued on the GPU, with route_check_torch's arguments (serve_route.py:141-184):
    logits [M, E] (fp32 / bf16 / fp16; other dtypes are widened to fp32), topk_w and topk_ids [M, k] as the router
    returned them, rows_buf[0] the step's real rows, stepbuf[0] the step, state[slot] the router's COLS counters,
    cap_*[slot] its kept row.  Computes only when the step is this router's turn."""
    from . import _lib
    m, e = int(logits.shape[0]), int(logits.shape[-1])
    if m == 0 or topk_ids.shape[0] < m:
        return
    _lib.require_gpu(logits, topk_w, topk_ids, bias, rows_buf, stepbuf, state, cap_meta, cap_lg, cap_ids, cap_w)
    if logits.dim() != 2 or topk_w.dim() != 2 or topk_ids.dim() != 2:
        raise ValueError("router logits, weights and ids must be 2-D")
    k = int(k)
    if topk_w.shape[0] < m or min(topk_w.shape[1], topk_ids.shape[1]) < k:
        raise ValueError(f"router weights {tuple(topk_w.shape)} / ids {tuple(topk_ids.shape)} for {m} rows of top-{k}")
    if state.dtype != torch.int64 or state.shape[-1] < COLS or state.stride(-1) != 1 or \
            cap_meta.dtype != torch.int64 or cap_meta.shape[-1] < CAP_COLS or cap_meta.stride(-1) != 1 or \
            cap_lg.dtype != torch.float32 or cap_lg.shape[-1] < e or cap_lg.stride(-1) != 1 or \
            cap_ids.dtype != torch.int64 or cap_ids.shape[-1] < k or cap_ids.stride(-1) != 1 or \
            cap_w.dtype != torch.float32 or cap_w.shape[-1] < k or cap_w.stride(-1) != 1:
        raise ValueError("the router's state row or kept-row tensors are too small for this call")
    if not (0 <= int(slot) < state.shape[0] and int(slot) < min(cap_meta.shape[0], cap_lg.shape[0],
                                                                  cap_ids.shape[0], cap_w.shape[0])):
        raise ValueError(f"slot {slot} is outside the state and kept-row tensors")
    if rows_buf.dtype != torch.int64 or stepbuf.dtype != torch.int64 or rows_buf.numel() < 1 or stepbuf.numel() < 1:
        raise ValueError("rows_buf and stepbuf are int64 words")
    lg = _last_dense(logits if logits.dtype in DTYPE_CODE else logits.float())
    w = _last_dense(topk_w if topk_w.dtype in _WEIGHT_DTYPES else topk_w.float())
    ids = _last_dense(topk_ids if topk_ids.dtype in _ID_CODE else topk_ids.long())
    b = None
    if bias is not None:
        b = bias if bias.dtype == torch.float32 and bias.is_contiguous() else bias.float().contiguous()
        if b.numel() != e:
            raise ValueError(f"a correction bias of {b.numel()} for {e} experts")
    L = _lib.lib()
    rc = L.sdc_route_check(lg.data_ptr(), lg.stride(0), DTYPE_CODE[lg.dtype], w.data_ptr(), w.stride(0),
                           DTYPE_CODE[w.dtype], ids.data_ptr(), ids.stride(0), _ID_CODE[ids.dtype], _lib.ptr(b), m, e,
                           k, int(scoring), int(bool(renormalize)), int(groups), int(topk_group), float(scale),
                           unit_roundoff(lg.dtype), rows_buf.data_ptr(), stepbuf.data_ptr(), max(int(nlayers), 1),
                           int(index), state[slot].data_ptr(), cap_meta[slot].data_ptr(), cap_lg[slot].data_ptr(),
                           cap_ids[slot].data_ptr(), cap_w[slot].data_ptr(), _lib.stream_of(lg))
    _lib.check(rc, "sdc_route_check")


route_check_torch = route_check          # the reference's names for the same call (one implementation here)
route_check_triton = route_check
route_check_any = route_check

_OP_LOCK = threading.Lock()
_OP: list = [None]


def route_op():
    """The check as one opaque op for torch.compile, registered once under the reference's name
    (sdcguard::route_check); where the op cannot be registered, the library call."""
    with _OP_LOCK:
        if _OP[0] is not None:
            return _OP[0]
        op = getattr(getattr(torch.ops, "sdcguard", None), "route_check", None)
        if op is None:
            try:
                lib_op = torch.library.custom_op(
                    "sdcguard::route_check", mutates_args=("state", "cap_meta", "cap_lg", "cap_ids", "cap_w"))(
                        _op_body)
                lib_op.register_fake(lambda *a: None)
                op = torch.ops.sdcguard.route_check
            except (AttributeError, RuntimeError):
                op = route_check
        _OP[0] = op
        return op


def _op_body(logits: torch.Tensor, topk_w: torch.Tensor, topk_ids: torch.Tensor, k: int, scoring: int,
             renormalize: bool, bias: Optional[torch.Tensor], groups: int, topk_group: int, scale: float,
             rows_buf: torch.Tensor, stepbuf: torch.Tensor, state: torch.Tensor, slot: int, nlayers: int, index: int,
             cap_meta: torch.Tensor, cap_lg: torch.Tensor, cap_ids: torch.Tensor, cap_w: torch.Tensor) -> None:
    route_check(logits, topk_w, topk_ids, k, scoring, renormalize, bias, groups, topk_group, scale, rows_buf,
                stepbuf, state, slot, nlayers, index, cap_meta, cap_lg, cap_ids, cap_w)


def check_call(binding, router_logits, topk_weights, topk_ids) -> None:
    """After one call of a registered router (select_experts): its logits and its result.  binding: the router's
    _sdcguard_route (set by RouteChecks.finalize)."""
    if binding is None or not all(isinstance(t, torch.Tensor) for t in (router_logits, topk_weights, topk_ids)):
        return
    args = binding.checks.call_args(binding)
    if router_logits.dim() != 2 or topk_ids.dim() != 2 or topk_ids.shape[-1] != args[0]:
        return
    call = (router_logits, topk_weights, topk_ids, *args)
    if torch.compiler.is_compiling():
        route_op()(*call)
        return
    with torch.no_grad():
        route_check(*call)


# ------------------------------------------------------------------------------------------------- the routers
_ROUTERS = {
    # class name: (groups read from the router, scaled by routed_scaling_factor)
    "FusedTopKRouter": (False, False),
    "FusedTopKBiasRouter": (False, True),
    "GroupedTopKRouter": (True, True),
}
_NOT_MODELED = ("_hash_indices_table", "bias_vl")     # hash routing, image-token biases


def _int(router, name: str) -> int:
    return int(getattr(router, name, 0) or 0)


def policy_of(router) -> tuple:
    """(policy, None) for a vLLM router the check models, or (None, why not).  The policy: k, scoring (0 softmax,
    1 sigmoid), renormalize, bias (a tensor or None), groups (0: plain top-k), topk_group, scale, experts (0 when the
    router does not say)."""
    kind = type(router).__name__
    if kind not in _ROUTERS:
        return None, f"the {kind} router (the check models vLLM's top-k, biased top-k and grouped top-k routers)"
    grouped, scaled = _ROUTERS[kind]
    scoring = str(getattr(router, "scoring_func", "softmax"))
    if scoring not in SCORING:
        return None, f"scoring function {scoring}"
    if getattr(router, "eplb_state", None) is not None:
        return None, "expert load balancing (the router returns physical expert ids)"
    if any(getattr(router, a, None) is not None for a in _NOT_MODELED) or _int(router, "num_fused_shared_experts"):
        return None, "hash routing, image-token biases or fused shared experts"
    k, e = _int(router, "top_k"), _int(router, "global_num_experts")
    if not 0 < k <= MAX_K or (e and (e > MAX_EXPERTS or k > e)):
        return None, f"top-{k} of {e} experts (the check takes up to top-{MAX_K} of {MAX_EXPERTS})"
    bias = getattr(router, "e_score_correction_bias", None)
    bias = getattr(bias, "data", bias)
    bias = bias if isinstance(bias, torch.Tensor) else None
    scale = float(getattr(router, "routed_scaling_factor", 1.0) or 1.0) if scaled else 1.0
    groups = _int(router, "num_expert_group") if grouped else 0
    topk_group = _int(router, "topk_group") if groups else 0
    if groups and not (e > groups and e % groups == 0):
        # a grouped router without a grouping of its experts routes as plain top-k; with no bias, that is the
        # fused top-k with softmax scores and no scaling, whatever its own settings say
        groups = topk_group = 0
        if bias is None:
            scoring, scale = "softmax", 1.0
    if groups and (groups > MAX_GROUPS or not 0 < topk_group <= groups or topk_group * (e // groups) < k):
        return None, f"{groups} expert groups choosing {topk_group}"
    return {"k": k, "scoring": SCORING[scoring], "renormalize": bool(getattr(router, "renormalize", True)),
            "bias": bias, "groups": groups, "topk_group": topk_group, "scale": scale, "experts": e}, None


def recheck(lg_row: torch.Tensor, ids: torch.Tensor, w: torch.Tensor, policy: dict, dtype: torch.dtype,
            device) -> dict:
    """The kept row judged again, alone, by the same kernel (the logits back in the dtype the router got them, which
    the widened kept copy holds exactly): output_wrong when it is wrong again, output_agrees when not (the check
    disagreed when the row ran in its batch)."""
    dev = torch.device(device)
    k, e = int(ids.numel()), int(lg_row.numel())
    lg = lg_row.reshape(1, e).to(dev).to(dtype)
    st = torch.zeros(1, COLS, dtype=torch.int64, device=dev)
    meta = torch.zeros(1, CAP_COLS, dtype=torch.int64, device=dev)
    clg = torch.zeros(1, e, device=dev)
    cid = torch.zeros(1, k, dtype=torch.int64, device=dev)
    cw = torch.zeros(1, k, device=dev)
    one = torch.ones(1, dtype=torch.int64, device=dev)
    zero = torch.zeros(1, dtype=torch.int64, device=dev)
    bias = policy["bias"].to(dev) if policy["bias"] is not None else None
    route_check(lg, w.reshape(1, k).to(dev).float(), ids.reshape(1, k).to(dev).long(), k, policy["scoring"],
                policy["renormalize"], bias, policy["groups"], policy["topk_group"], policy["scale"], one, zero, st, 0,
                1, 0, meta, clg, cid, cw)
    keys = [int(v) for v in st[0].cpu().tolist()]
    out = {"experts": [int(v) for v in ids.tolist()], "weights": [float(v) for v in w.tolist()],
           "worst_weight_difference": f32_of(keys[C_WDIFF])}
    # both samples of a one-row call are the row: each finding counts twice
    if keys[C_SET] or keys[C_WEIGHT]:
        what = "experts" if keys[C_SET] else "weights"
        return {**out, "verdict": "output_wrong",
                "why": f"judged again alone from the kept logits, the router's {what} are wrong for its policy"}
    return {**out, "verdict": "output_agrees",
            "why": "judged again alone from the kept logits, the router's experts and weights fit its policy: the "
                   "check disagreed when the row ran in its batch"}


class RouteChecks(StepChecks):
    """The MoE routers one ServeGuard checks (ServeGuard.route_checks()): add() each at load, finalize() after the
    last and before any graph is captured (it numbers the routers' turns and binds them), mark_step() / end_step()
    around each model step, poll() to read."""

    DETECTOR = "serve_route"
    COLS = COLS
    CAPTURE = {"meta": torch.int64, "lg": torch.float32, "ids": torch.int64, "w": torch.float32}
    READ_CAPTURE = ()

    def __init__(self, guard=None):
        super().__init__(guard)
        self.finalized = False
        self.stats.update(calls=0, rows=0, wrong_sets=0, wrong_weights=0)

    def add(self, router, name: str, device) -> Optional[int]:
        """Register a router (before finalize()); returns its slot, or None when the check does not model it."""
        if self.finalized:
            raise RuntimeError("routers are added before finalize()")
        if getattr(router, "_sdcguard_route", None) is not None:
            self._refuse(name, "already checked by another ServeGuard")
            return None
        pol, why = policy_of(router)
        if why:
            self._refuse(name, why)
            return None
        device = torch.device(device)
        if device.type != "cuda":
            self._refuse(name, "not on a GPU")
            return None
        if pol["bias"] is not None:
            with torch.inference_mode(False), torch.no_grad():
                b = pol["bias"]
                pol["bias"] = b if b.device == device and b.dtype == torch.float32 and b.is_contiguous() else \
                    b.detach().to(device, torch.float32).contiguous()
        e = pol["experts"] or MAX_EXPERTS
        b = self._register(name, router, device, widths={"meta": CAP_COLS, "lg": e, "ids": pol["k"], "w": pol["k"]},
                           policy=pol)
        return b.slot

    def finalize(self) -> int:
        """Number each device's routers' turns, register the op and give each router its binding."""
        if self.finalized:
            return len(self.layers)
        per_dev: dict = {}
        for lay in self.layers:
            per_dev.setdefault(lay.device, []).append(lay)
        for lays in per_dev.values():
            for turn, lay in enumerate(lays):
                lay.info["index"], lay.info["nlayers"] = turn, len(lays)
        route_op()
        for n, lay in enumerate(self.layers):
            lay.module._sdcguard_route = Binding(self, n)
        self.finalized = True
        return len(self.layers)

    def call_args(self, b: Binding) -> tuple:
        """The library call's arguments after (logits, topk_w, topk_ids) for a binding's router."""
        lay, tab = b.layer, b.table()
        p, c = lay.info["policy"], tab.capture
        return (p["k"], p["scoring"], p["renormalize"], p["bias"], p["groups"], p["topk_group"], p["scale"],
                tab.word.view(W_ROWS), tab.word.view(W_STEP), tab.state, lay.slot, lay.info["nlayers"],
                lay.info["index"], c["meta"], c["lg"], c["ids"], c["w"])

    def detach(self) -> None:
        super().detach()
        self.finalized = False

    def _unbind(self, lay: Registered) -> None:
        lay.module.__dict__.pop("_sdcguard_route", None)

    def coverage(self) -> dict:
        out = super().coverage()
        out.update(calls=self.stats["calls"], rows=self.stats["rows"], samples_per_call=SAMPLES,
                   one_router_a_step=True)
        return out

    def _count(self, lay: Registered, k: list) -> None:
        lay.calls += k[C_CALLS]
        for stat, col in (("calls", C_CALLS), ("rows", C_ROWS), ("wrong_sets", C_SET), ("wrong_weights", C_WEIGHT)):
            self.stats[stat] += k[col]
        if k[C_WDIFF]:
            lay.worst = max(lay.worst, f32_of(k[C_WDIFF]))

    def _judged(self, k: list) -> bool:
        return k[C_ROWS] > 0

    def _judge(self, lay: Registered, k: list, captured: dict, window) -> list:
        if not (k[C_SET] or k[C_WEIGHT]):
            return []
        from .serve_fp8 import unwrap31
        last = k[C_LAST]
        kind, row = (last >> 24) & 0xFF, last & 0xFFFFFF
        step = unwrap31(last >> 32, self.marked)
        finding = "wrong_experts" if kind == KIND_SET else "wrong_weights"
        pol = {kk: v for kk, v in lay.info["policy"].items() if kk != "bias"}
        pol["bias"] = lay.info["policy"]["bias"] is not None
        detail = {"where": lay.name, "kind": "moe_routing", "finding": finding, "rows_judged": k[C_ROWS],
                  "rows_with_wrong_experts": k[C_SET], "rows_with_wrong_weights": k[C_WEIGHT],
                  "worst_weight_difference": f32_of(k[C_WDIFF]) if k[C_WDIFF] else 0.0,
                  "captured": {"step": step if self.marked is not None else None, "row": row}, "policy": pol,
                  "read_window_steps": window, "last_clean_read_steps": self.last_clean(lay.name),
                  "reading": ("the router chose experts its policy does not give for these logits"
                              if finding == "wrong_experts" else
                              "the router's weights for its experts differ from its policy's")}
        detail["recheck"] = self._recheck(lay)
        return [self.emit(lay, math.inf, row, detail)]

    def _recheck(self, lay: Registered) -> dict:
        """The router's kept row (its first wrong row since the last read) judged again; its capture is freed."""
        c = self.tables[lay.device].capture
        meta = [int(v) for v in c["meta"][lay.slot].tolist()]
        if not meta[0]:
            return {"verdict": "not_rechecked", "why": "no row was kept (an earlier alert's kept row was read first)"}
        e, k = meta[4], lay.info["policy"]["k"]
        try:
            out = recheck(c["lg"][lay.slot, :e].clone(), c["ids"][lay.slot, :k].clone(),
                          c["w"][lay.slot, :k].clone(), lay.info["policy"], CODE_DTYPE.get(meta[5], torch.float32),
                          lay.device)
            out["captured"] = {"row": meta[1], "step": meta[2] if self.marked is not None else None,
                               "kind": "experts" if meta[3] == KIND_SET else "weights"}
        except Exception as ex:  # noqa: BLE001  (the diagnosis is best effort)
            out = {"verdict": "not_rechecked", "why": f"{type(ex).__name__}: {ex}"}
        c["meta"][lay.slot].zero_()
        return out
