"""Training-side checks: Group, check_now and SDCGuard (reference: _group.py:749-917, guard.py:788-1971).

Group gathers the checks of one step on one device and dtype: add() queues a check's GPU work at once
(sdc_matmul_check: the block sums of B, the expected side on MFMA, one scoring pass over C that leaves the check's
worst key in a device row); launch() collects every check's row into one device tensor; a single device-to-host copy
per flush then reads them all, and row() decodes one.  check_now() is one check answered right away.

SDCGuard checks the nn.Linear layers of a model while a step is active (protect() + at_step()): each layer's
forward product y = x W^T + b, its input gradient dx = dy W and its weight gradient dW = dy^T x, on a share of
them (sample_rate), queued without host synchronisation and read back by flush() (every `every` steps, at
max_pending queued checks, or when called).  Alerts become SDCEvent records, call on_alert, and raise SDCError with
raise_on_alert.

precise=True (guard.py:31-35, :471-530): on checked steps each protected layer computes those three products with
an fp32 output (the accumulator), queues the precise check of it (matmul_zscores_acc: float64 checksums against the
fp32 accumulation's own rounding, far below what bf16 rounding hides), then rounds it once; on_accumulator(layer,
pass, C32) may change the fp32 result before its check (fault injection).  Unchecked steps run the layer unchanged.
precise="fused" (guard.py:1209-1270): the same products come from the library's fused GEMM, whose epilogue checks
the fp32 accumulator before rounding it (fused.fused_mm_checked; fused_mm + zscores_from_stats with
SDCGUARD_FUSED_FP64=1), so no fp32 product is written or read back; fused_inject(layer, pass, (m, n)) -> (row, col,
value) or None adds a fault to one accumulator element (experiments).  A product the fused kernel refuses switches
the guard to precise=True from then on (stats["fused_fallbacks"], fused_why).
SDCGuard(ops=True) adds the dispatch route (guard.py:1651-1805): on checked steps a TorchDispatchMode sees every
aten matmul of the step -- mm, addmm, bmm, baddbmm and torch._grouped_mm (MoE experts), in the forward pass and,
through the autograd engine's threads, the backward pass -- and queues its check with the same Group.  The MoE layout
(tokens x experts' weights, offs on the device) is checked by one grouped launch with the group ends read on the GPU;
the other grouped layouts are split per group on offs read on the host, as the reference splits them
(guard.py:102-143).  The reference's other routes (DTensor shards, replica and evidence capture) are not part of
this path.
"""
from __future__ import annotations

import contextlib
import math
import os
import random
import threading
import time
from dataclasses import dataclass, field
from typing import Callable, Optional

import torch

from torch.utils._python_dispatch import TorchDispatchMode

from .checksum import (ABS_FLOOR, UNIT_ROUNDOFF, CheckResult, _f32_of_bits, grouped_checks, grouped_zscores,
                       is_empty, matmul_zscores, matmul_zscores_acc, resolve_grouped)

UNJUDGED = -1.0


class Group:
    """The checks of one step on one device in one dtype (the reference's _group.Group interface)."""

    CHUNK = 256                         # result rows allocated at a time

    def __init__(self, device, dtype: torch.dtype, block: int = 128, abs_floor: float = ABS_FLOOR,
                 z: float = 6.0, epoch: int = 0, precise: bool = False, nfma: Optional[int] = None):
        """dtype: the outputs' (bf16 / fp16); with precise, the operands' (the outputs are their fp32 products,
        checked by matmul_zscores_acc with nfma products per tensor-core step)."""
        if dtype not in UNIT_ROUNDOFF:
            raise ValueError(f"checks take bf16 / fp16 {'operands' if precise else 'outputs'}, not {dtype}")
        self.device, self.dtype, self.block = torch.device(device), dtype, int(block)
        self.abs_floor, self.z, self.epoch = float(abs_floor), float(z), int(epoch)
        self.precise, self.nfma = bool(precise), nfma
        self.fused = False              # checks queued by add_fused (the fused GEMM's own)
        self.meta: list = []            # per check: (rows m, blocks nb, batched)
        self._rows: list = []           # (CHUNK, 3) int64 result blocks on the device
        self.result: Optional[torch.Tensor] = None

    def __len__(self) -> int:
        return len(self.meta)

    def _slot(self) -> torch.Tensor:
        i = len(self.meta)
        if i // self.CHUNK >= len(self._rows):
            self._rows.append(torch.zeros(self.CHUNK, 3, dtype=torch.int64, device=self.device))
        return self._rows[i // self.CHUNK][i % self.CHUNK]

    def add(self, A, B, C, bias, alpha: float, beta: float) -> int:
        """Check C = beta * bias + alpha * (A @ B): the GPU work is queued now.  Returns the check's index."""
        if self.precise:
            if C.dtype != torch.float32 or A.dtype != self.dtype:
                raise ValueError(f"this group checks fp32 products of {self.dtype}, not {A.dtype} -> {C.dtype}")
            st = matmul_zscores_acc(A, B, C, bias, alpha=alpha, beta=beta, block=self.block, abs_floor=self.abs_floor,
                                    z=self.z, nfma=self.nfma, epoch=self.epoch, out=self._slot())
        else:
            if C.dtype != self.dtype:
                raise ValueError(f"this group checks {self.dtype} outputs, not {C.dtype}")
            st = matmul_zscores(A, B, C, bias, alpha=alpha, beta=beta, block=self.block, abs_floor=self.abs_floor,
                                z=self.z, epoch=self.epoch, out=self._slot())
        self.meta.append((st.m, st.nb, st.batched))
        return len(self.meta) - 1

    def add_fused(self, A, B, bias, inject=None, fp64: bool = False):
        """C = A @ B + bias from the fused GEMM with the check of its fp32 accumulator queued here (fused.py);
        fp64: statistics scored in float64 (zscores_from_stats) instead of the kernel's own fp32 self-check.
        Returns (C rounded to A's dtype, the check's index)."""
        from . import fused as _fused
        if A.dtype != self.dtype:
            raise ValueError(f"this group checks products of {self.dtype}, not {A.dtype}")
        if fp64:
            C, stats = _fused.fused_mm(A, B, bias, epoch=self.epoch, inject=inject)
            st = _fused.zscores_from_stats(A, B, stats, bias, z=self.z, nfma=self.nfma, epoch=self.epoch,
                                           abs_floor=self.abs_floor, out=self._slot())
        else:
            C, st = _fused.fused_mm_checked(A, B, bias, z=self.z, nfma=self.nfma, epoch=self.epoch,
                                            abs_floor=self.abs_floor, inject=inject, out=self._slot())
        self.fused = True
        self.meta.append((st.m, st.nb, False))
        return C, len(self.meta) - 1

    def launch(self) -> None:
        """Every check's result row in one device tensor (checks, 3); never waits for the GPU."""
        n = len(self.meta)
        self.result = torch.cat(self._rows)[:n] if n else torch.zeros(0, 3, dtype=torch.int64, device=self.device)

    def row(self, idx: int, r) -> tuple:
        """Decode read-back row r (key, key with noise, unjudged) of check idx: (max_z, batch, row, col_block,
        noise); an incomplete check (unjudged checksums) that does not alarm reads -1, never clean."""
        m, nb, _batched = self.meta[idx]
        key, keyd, unjudged = (int(v) for v in r)
        z = _f32_of_bits(key >> 32)
        if unjudged and z <= self.z:
            z = UNJUDGED
        b_i, rem = divmod((key & 0xFFFFFFFF) // 2, m * nb)
        row, col_block = divmod(rem, nb)
        return z, b_i, row, col_block, _f32_of_bits(keyd)


def check_now(A, B, C, bias=None, alpha=1.0, beta=1.0, block=128, abs_floor=1e-20, z=6.0, epoch=0) -> tuple:
    """One check answered right away: (max_z, batch, row, col_block, noise)."""
    g = Group(C.device, C.dtype, block, abs_floor, z, epoch=epoch)
    g.add(A, B, C, bias, alpha, beta)
    g.launch()
    return g.row(0, g.result[0].tolist())


class SDCError(RuntimeError):
    """Raised by flush() when a check alarms and raise_on_alert is set."""


@dataclass
class SDCEvent:
    """One alert of the training guard."""
    detector: str
    layer: str
    z: float
    step: Optional[int] = None
    row: Optional[int] = None
    col_block: Optional[int] = None
    noise: Optional[float] = None
    nonfinite: bool = False
    time: float = field(default_factory=time.time)
    extra: dict = field(default_factory=dict)


def _acc_mm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a @ b of 16-bit operands with the fp32 result itself (guard.py:281-301), autocast off."""
    with torch.autocast(device_type=a.device.type, enabled=False):
        try:
            return torch.mm(a, b, out_dtype=torch.float32)
        except (RuntimeError, TypeError, NotImplementedError):
            saved = torch.backends.cuda.matmul.allow_tf32
            torch.backends.cuda.matmul.allow_tf32 = False
            try:
                return a.float() @ b.float()
            finally:
                torch.backends.cuda.matmul.allow_tf32 = saved


class _PreciseLinear(torch.autograd.Function):
    """y = x W^T + b on a checked step of precise mode: every product's fp32 result is checked, then rounded once
    (the bias added in fp32 first, as one GEMM with a bias epilogue does)."""

    @staticmethod
    def forward(ctx, x, w, b, guard, label):
        x2 = x.reshape(-1, x.shape[-1])
        ctx.save_for_backward(x, w)
        ctx.guard, ctx.label, ctx.has_bias = guard, label, b is not None
        y = guard._fused(label, "forward", x2, w.t(), b)
        if y is None:
            y32 = _acc_mm(x2, w.t())
            if b is not None:
                y32 = y32.add_(b.float())
            guard._accumulator(label, "forward", x2, w.t(), y32, b)
            y = y32.to(x.dtype)
        return y.view(*x.shape[:-1], w.shape[0])

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        guard, label = ctx.guard, ctx.label
        gy2 = gy.reshape(-1, gy.shape[-1]).to(x.dtype)
        x2 = x.reshape(-1, x.shape[-1])
        need_x, need_w, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        gx = gw = gb = None
        checked = guard._active
        if need_x:
            gx = guard._fused(label, "input grad", gy2, w, None) if checked else None
            if gx is None:
                gx32 = _acc_mm(gy2, w)
                if checked:
                    guard._accumulator(label, "input grad", gy2, w, gx32, None)
                gx = gx32.to(x.dtype)
            gx = gx.view(x.shape)
        if need_w:
            gyt = gy2.t()
            gw = guard._fused(label, "weight grad", gyt, x2, None) if checked else None
            if gw is None:
                gw32 = _acc_mm(gyt, x2)
                if checked:
                    guard._accumulator(label, "weight grad", gyt, x2, gw32, None)
                gw = gw32
            gw = gw.to(w.dtype)
        if need_b and ctx.has_bias:
            gb = gy2.sum(0)
        return gx, gw, gb, None, None


# ------------------------------------------------------------------------------------------ the dispatch route
def _scales(args, kwargs) -> tuple:
    """(alpha, beta) of an addmm / baddbmm call: beta scales the added input, alpha the product."""
    beta = kwargs.get("beta", args[3] if len(args) > 3 else 1)
    alpha = kwargs.get("alpha", args[4] if len(args) > 4 else 1)
    return float(alpha), float(beta)


# aten op -> its product C = beta * bias + alpha * (A @ B) as (A, B, C, bias, alpha, beta); the products the
# reference's matmul_checks (guard.py:222-264) takes for these ops
_OP_PRODUCTS = {
    "mm": lambda a, kw, out: (a[0], a[1], out, None, 1.0, 1.0),
    "bmm": lambda a, kw, out: (a[0], a[1], out, None, 1.0, 1.0),
    "addmm": lambda a, kw, out: (a[1], a[2], out, a[0], *_scales(a, kw)),
    "baddbmm": lambda a, kw, out: (a[1], a[2], out, a[0], *_scales(a, kw)),
}


def _grouped_args(args, kwargs) -> tuple:
    """(a, b, offs, bias) of a torch._grouped_mm call."""
    offs = kwargs.get("offs", args[2] if len(args) > 2 else None)
    bias = kwargs.get("bias", args[3] if len(args) > 3 else None)
    return args[0], args[1], offs, bias


class _OpWatch(TorchDispatchMode):
    """The guard's view of every aten operator while a checked step runs: matmul results are handed to the guard
    after the operator ran (this mode is paused inside its own handler, so the checks' own operators pass by)."""

    def __init__(self, guard: "SDCGuard"):
        super().__init__()
        self.guard = guard

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        out = func(*args, **kwargs)
        name = func.overloadpacket.__name__
        if (name in _OP_PRODUCTS or name == "_grouped_mm") and self.guard._active:
            self.guard._op_result(name, args, kwargs, out)
        return out


def _plain_linear(mod: torch.nn.Module) -> bool:
    return isinstance(mod, torch.nn.Linear) and type(mod).forward is torch.nn.Linear.forward and \
        "forward" not in mod.__dict__


class SDCGuard:
    """Checksums the matmuls of a model's linear layers on sampled steps (the reference's SDCGuard, protect() mode).

        guard = SDCGuard().protect(model)
        for step, batch in enumerate(data):
            with guard.at_step(step):
                loss = model(batch).sum()
                loss.backward()
        guard.flush()
    """

    def __init__(self, sample_rate: float = 1.0, block: int = 128, z: float = 6.0,
                 on_alert: Optional[Callable[[SDCEvent], None]] = None, raise_on_alert: bool = False,
                 abs_floor: Optional[float] = None, every: int = 10, max_pending: int = 4096,
                 fresh_signs: bool = True, seed: int = 0, precise=False, nfma: Optional[int] = 16,
                 on_accumulator: Optional[Callable[[str, str, torch.Tensor], None]] = None, recompute: bool = False,
                 ops: bool = False):
        """precise: True or "fused", check the fp32 accumulators of the protected layers' products (see the module
        docstring); nfma: products per tensor-core accumulation step of those products (16: one 32x32x16 MFMA;
        None: none); recompute: also compare each activation-checkpointed block's recompute with its forward run
        (recompute.RecomputeCheck, installed by protect() and flushed with the checks); ops: check every aten
        matmul of a checked step (mm, addmm, bmm, baddbmm, torch._grouped_mm) through a dispatch mode instead of the
        protected layers' hooks (protect() then only installs the recompute check)."""
        if not 0.0 <= sample_rate <= 1.0:
            raise ValueError("sample_rate is a share in [0, 1]")
        if precise not in (False, True, "fused"):
            raise ValueError(f"precise is False, True or 'fused', not {precise!r}")
        if ops and precise:
            raise ValueError("the dispatch route checks bf16 / fp16 results as they are (precise needs the layers' "
                             "fp32 products)")
        self.ops = bool(ops)
        self.ops_seen: dict = {}            # aten matmul -> calls seen on checked steps (the dispatch route)
        self.sample_rate, self.block, self.z = float(sample_rate), int(block), float(z)
        self.on_alert, self.raise_on_alert = on_alert, raise_on_alert
        self.abs_floor = ABS_FLOOR if abs_floor is None else float(abs_floor)
        self.every, self.max_pending, self.fresh_signs = int(every), int(max_pending), fresh_signs
        self.precise, self.nfma, self.on_accumulator = precise, nfma, on_accumulator
        self.fused_inject: Optional[Callable] = None      # precise="fused": (layer, pass, (m, n)) -> fault or None
        self._fused_off = False                           # the fused kernel refused a product: precise=True now
        self.fused_why: Optional[str] = None
        self.recompute = None
        if recompute:
            from .recompute import RecomputeCheck
            self.recompute = RecomputeCheck(on_alert=self._recompute_alert)
        self._rng = random.Random(seed)
        self._lock = threading.RLock()
        self._hooks: list = []
        self._protected: list = []
        self._active = False
        self.step: Optional[int] = None
        self._epoch = 0
        self._groups: dict = {}             # (device, dtype) -> Group of the open checks
        self._wctx: dict = {}               # id(layer) -> what its weight-gradient check needs, this step
        self._pending: list = []            # (group, index, layer, pass, step)
        self.events: list = []
        self.results: list = []
        self.stats = {"layers": 0, "matmuls_seen": 0, "checks": 0, "alerts": 0, "skipped_dtype": 0, "flushes": 0}
        if precise == "fused":
            self.stats.update(checked_fused=0, fused_fallbacks=0)

    # ------------------------------------------------------------------------------------------- protect
    def _recompute_alert(self, ev) -> None:
        rec = SDCEvent(detector="recompute", layer=ev.layer, z=ev.z, step=self.step, extra=dict(ev.extra))
        self.events.append(rec)
        self.stats["alerts"] += 1
        if self.on_alert is not None:
            self.on_alert(rec)

    def protect(self, model: torch.nn.Module) -> "SDCGuard":
        """Check the forward product and both gradient products of every plain nn.Linear of `model`."""
        if self.recompute is not None:
            self.recompute.install(model)
        if self.ops:                         # (the dispatch route sees every product itself)
            return self
        for name, mod in model.named_modules():
            if not _plain_linear(mod) or mod in self._protected:
                continue
            label = name or type(mod).__name__
            self._protected.append(mod)
            if self.precise:
                mod.forward = self._precise_forward(mod, label)
            else:
                self._hooks.append(mod.register_forward_hook(self._after_forward(label)))
                self._hooks.append(mod.register_full_backward_hook(self._after_backward(label)))
            self.stats["layers"] += 1
        return self

    def unprotect(self) -> None:
        if self.recompute is not None:
            self.recompute.uninstall()
        for h in self._hooks:
            h.remove()
        self._hooks.clear()
        for mod in self._protected:
            mod.__dict__.pop("forward", None)
        self._protected.clear()

    def _precise_forward(self, mod: torch.nn.Module, label: str):
        linear = torch.nn.functional.linear

        def forward(x):
            w, b = mod.weight, mod.bias
            if not self._active or not x.is_cuda:
                return linear(x, w, b)
            if torch.is_autocast_enabled("cuda"):
                dt = torch.get_autocast_dtype("cuda")
                x, w, b = x.to(dt), w.to(dt), (None if b is None else b.to(dt))
            if x.dtype not in UNIT_ROUNDOFF or w.dtype != x.dtype:
                self.stats["skipped_dtype"] += 1
                return linear(x, w, b)
            grads = torch.is_grad_enabled()              # the forward, and each gradient product backward will run
            self.stats["matmuls_seen"] += 1 + int(grads and x.requires_grad) + int(grads and w.requires_grad)
            with torch.autocast(device_type="cuda", enabled=False):
                return _PreciseLinear.apply(x, w, b, self, label)
        return forward

    def _fused(self, layer: str, where: str, A, B, bias):
        """precise="fused": A @ B (+ bias) from the fused GEMM with its check queued, or None where the fused
        kernel does not take it (the caller computes the fp32 product and checks it as precise=True does).  A product
        left out by sample_rate is the ordinary matmul, unchecked."""
        if self.precise != "fused" or self._fused_off or not A.is_cuda:
            return None
        if A.shape[0] == 0 or A.shape[1] == 0 or B.shape[1] == 0:
            return None
        if not self._sampled():
            C = A @ B.to(A.dtype)
            return C if bias is None else C.add_(bias.to(C.dtype))
        inj = self.fused_inject(layer, where, (A.shape[0], B.shape[1])) if self.fused_inject is not None else None
        from ._lib import HipLibraryError
        with self._lock:
            key = (A.device, A.dtype, "fused")
            g = self._groups.get(key)
            if g is None:
                g = self._groups[key] = Group(A.device, A.dtype, self.block, self.abs_floor, self.z, self._epoch,
                                              precise=True, nfma=self.nfma)
            try:
                C, i = g.add_fused(A, B, bias, inject=inj, fp64=os.environ.get("SDCGUARD_FUSED_FP64") == "1")
            except HipLibraryError as e:
                self._fused_off = True
                self.stats["fused_fallbacks"] += 1
                self.fused_why = f"{layer} ({where}): {e}"
                import warnings
                warnings.warn(f"the fused precise check refused a product, precise=True takes over: {self.fused_why}",
                              RuntimeWarning, stacklevel=2)
                return None
            self._pending.append((g, i, layer, where, self.step, None))
            self.stats["checks"] += 1
            self.stats["checked_fused"] += 1
        return C

    def _accumulator(self, layer: str, where: str, A, B, C32, bias) -> None:
        """Precise mode: one product's fp32 result before it is rounded (on_accumulator may change it first)."""
        if self.on_accumulator is not None:
            self.on_accumulator(layer, where, C32)
        if C32.numel() == 0 or not self._sampled():
            return
        with self._lock:
            key = (C32.device, A.dtype, "fp32")
            g = self._groups.get(key)
            if g is None:
                g = self._groups[key] = Group(C32.device, A.dtype, self.block, self.abs_floor, self.z, self._epoch,
                                              precise=True, nfma=self.nfma)
            i = g.add(A, B, C32, bias, 1.0, 1.0)
            self._pending.append((g, i, layer, where, self.step, None))
            self.stats["checks"] += 1

    def _sampled(self) -> bool:
        return self.sample_rate >= 1.0 or self._rng.random() < self.sample_rate

    def _after_forward(self, label: str):
        def hook(mod, args, y):
            if not self._active or not args or not torch.is_tensor(y):
                return None
            x = args[0]
            self.stats["matmuls_seen"] += 1
            if self._sampled():
                x2, y2 = x.reshape(-1, x.shape[-1]), y.reshape(-1, y.shape[-1])
                self._queue(label, "forward", x2, mod.weight.t(), y2, mod.bias)
            w = mod.weight
            if y.requires_grad and w.requires_grad:
                # the weight-gradient check needs x and dy; a layer used twice in a step gets the sum of two
                # products as its weight gradient, which one (x, dy) pair does not check: it is left out
                prev = self._wctx.get(id(mod))
                if prev is not None:
                    prev["shared"] = True
                    return None
                ctx = {"x": x.detach()}
                self._wctx[id(mod)] = ctx
                y.register_hook(lambda g, ctx=ctx: ctx.__setitem__("dy", g))
                ctx["whook"] = w.register_hook(lambda gw, ctx=ctx: self._weight_grad(label, ctx, gw))
            return None
        return hook

    def _weight_grad(self, label: str, ctx: dict, gw: torch.Tensor):
        h = ctx.pop("whook", None)
        if h is not None:
            h.remove()
        dy = ctx.get("dy")
        if dy is None or ctx.get("shared") or not self._active:
            return None
        self.stats["matmuls_seen"] += 1
        if self._sampled():
            dy2 = dy.reshape(-1, dy.shape[-1])
            x2 = ctx["x"].reshape(-1, ctx["x"].shape[-1])
            self._queue(label, "weight grad", dy2.t().contiguous(), x2, gw, None)
        return None

    def _after_backward(self, label: str):
        def hook(mod, grad_input, grad_output):
            if not self._active or not grad_input or grad_input[0] is None or grad_output[0] is None:
                return None
            self.stats["matmuls_seen"] += 1
            if self._sampled():
                gx, gy = grad_input[0], grad_output[0]
                self._queue(label, "input grad", gy.reshape(-1, gy.shape[-1]), mod.weight,
                            gx.reshape(-1, gx.shape[-1]), None)
            return None
        return hook

    def _queue(self, layer: str, where: str, A, B, C, bias, alpha: float = 1.0, beta: float = 1.0,
               extra: Optional[dict] = None) -> None:
        """Queue one check of C = beta * bias + alpha * (A @ B): its GPU work starts now; the result is read at the
        flush."""
        if C.dtype not in UNIT_ROUNDOFF or not C.is_cuda:
            self.stats["skipped_dtype"] += 1
            return
        if C.numel() == 0:
            return
        with self._lock:
            key = (C.device, C.dtype)
            g = self._groups.get(key)
            if g is None:
                g = self._groups[key] = Group(C.device, C.dtype, self.block, self.abs_floor, self.z, self._epoch)
            i = g.add(A, B, C, bias, alpha, beta)
            self._pending.append((g, i, layer, where, self.step, extra))
            self.stats["checks"] += 1

    def _op_result(self, name: str, args, kwargs, out) -> None:
        """The dispatch route: one aten matmul's result, seen on a checked step (forward or backward)."""
        node = torch._C._current_autograd_node()
        where = f"backward ({node.name()})" if node is not None else "forward"
        label = f"aten.{name}"
        with self._lock:
            self.stats["matmuls_seen"] += 1
            self.ops_seen[label] = self.ops_seen.get(label, 0) + 1
        if not self._sampled():
            return
        if name != "_grouped_mm":
            A, B, C, bias, alpha, beta = _OP_PRODUCTS[name](args, kwargs, out)
            self._queue(label, where, A, B, C, bias, alpha, beta,
                        extra={"op": label, "shape_A": tuple(A.shape), "shape_B": tuple(B.shape)})
            return
        a, b, offs, bias = _grouped_args(args, kwargs)
        if not out.is_cuda or out.dtype not in UNIT_ROUNDOFF:
            self.stats["skipped_dtype"] += 1
            return
        if a.dim() == 2 and b.dim() == 3 and offs is not None and (bias is None or bias.numel() == out.shape[-1]):
            # tokens sorted by expert: one grouped launch, the group ends read on the GPU
            st = grouped_zscores(a, b, out, offs, bias, block=self.block, abs_floor=self.abs_floor, z=self.z,
                                 epoch=self._epoch)
            with self._lock:
                self._pending.append((None, st, label, where, self.step,
                                      {"op": label, "shape_A": tuple(a.shape), "shape_B": tuple(b.shape)}))
                self.stats["checks"] += 1
            return
        for gi, (A, B, C, bi, al, be) in enumerate(grouped_checks(a, b, out, offs, bias)):
            if not is_empty(C):
                self._queue(label, where, A, B, C, bi, al, be,
                            extra={"op": label, "group": gi, "shape_A": tuple(A.shape), "shape_B": tuple(B.shape)})

    # ------------------------------------------------------------------------------------------- steps
    @contextlib.contextmanager
    def at_step(self, step: int):
        """Check the protected layers' matmuls of this step (a nested call does nothing: the outer step counts)."""
        if self._active:
            yield self
            return
        self.step = int(step)
        if self.fresh_signs:
            self._epoch = self.step + 1        # a new signed-checksum pattern every checked step
        self._active = True
        watch = _OpWatch(self) if self.ops else contextlib.nullcontext()
        try:
            with watch:
                yield self
        finally:
            self._active = False
            for ctx in self._wctx.values():          # (a forward whose backward did not run this step)
                h = ctx.pop("whook", None)
                if h is not None:
                    h.remove()
            self._wctx.clear()
            with self._lock:
                self._groups = {}                    # the next step's checks use its own sign pattern
            if len(self._pending) >= self.max_pending or (self.every > 0 and self.step % self.every == 0):
                self.flush()

    def flush(self) -> list:
        """Read every queued check back (one device-to-host copy per device), record the results and raise alerts.
        Returns their CheckResults in queue order."""
        if self.recompute is not None:
            self.recompute.step = self.step
            self.recompute.flush()
        with self._lock:
            pending, self._pending = self._pending, []
            groups = {id(g): g for g, *_ in pending if g is not None}
            self._groups = {}
        if not pending:
            return []
        self.stats["flushes"] += 1
        by_dev: dict = {}
        for g in groups.values():
            g.launch()
            by_dev.setdefault(g.device, []).append(g)
        rows = {}
        for gs in by_dev.values():
            back = torch.cat([g.result for g in gs]).cpu().tolist()
            i = 0
            for g in gs:
                rows[id(g)] = back[i:i + len(g)]
                i += len(g)
        out, alerts = [], []

        def judge(res, g, layer, where, step, info, batch=None, group=None):
            out.append(res)
            if res.ok:
                return
            extra = {"pass": where, **(info or {})}
            if batch is not None:
                extra["batch"] = batch
            if group is not None:
                extra["group"] = group
            if g is not None and g.fused:
                extra["dtype"] = f"float32 accumulator of {g.dtype} (fused)"
            alerts.append(SDCEvent(detector="accumulator" if g is not None and g.precise else "checksum",
                                   layer=layer, z=res.max_z, step=step, row=res.row, col_block=res.col_block,
                                   noise=res.noise, nonfinite=res.nonfinite, extra=extra))

        for g, i, layer, where, step, info in pending:
            if g is None:                        # a grouped launch: one result per non-empty group, in group order
                st, start, nonempty = i, 0, []
                for gi, e in enumerate(int(v) for v in st.offs.tolist()):
                    e = min(e, st.rows)
                    if e > start:
                        nonempty.append(gi)
                    start = max(start, e)
                for gi, res in zip(nonempty, resolve_grouped(st)):
                    judge(res, None, layer, where, step, info, group=gi)
                continue
            z, b_i, r_i, c_i, noise = g.row(i, rows[id(g)][i])
            finite = math.isfinite(z)
            res = CheckResult(ok=finite and z <= self.z, max_z=z, nonfinite=not finite, batch=None, row=r_i,
                              col_block=c_i, noise=noise)
            judge(res, g, layer, where, step, info, batch=b_i if g.meta[i][2] else None)
        self.results.extend(out)
        for ev in alerts:
            self.events.append(ev)
            self.stats["alerts"] += 1
            if self.on_alert is not None:
                self.on_alert(ev)
        if alerts and self.raise_on_alert:
            a = alerts[0]
            raise SDCError(f"silent data corruption suspected: {a.layer} ({a.extra['pass']}) at step {a.step}, "
                           f"z = {a.z:.3g}, row {a.row}, column block {a.col_block}")
        return out
