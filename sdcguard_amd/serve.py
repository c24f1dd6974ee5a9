"""Serving check: every bf16/fp16 linear layer on every forward pass (reference: serve.py).

Weights do not change while a model serves, so each layer's block sums are computed once (LayerChecksums, built on
the GPU by sdc_layer_constants) and every forward pass only reads the layer's input x and output y again:

    expected = x @ (block sums of W)       MFMA, three low-precision parts of the fp32 sums
    actual   = block sums of y             one pass over y
    z        = |expected - actual| / rounding noise,  fault above z (default 6)

The work runs in libsdcguard_hip.so (sdc_check_static), no host synchronisation; the worst score goes into a
per-layer int64 state row with atomic maxima and is read back asynchronously by ServeGuard.poll().  The custom op
sdcguard::check_static keeps the reference's argument list (serve.py:465-489), so torch.compile sees one opaque call
and HIP graphs capture its kernels.
"""
from __future__ import annotations

import math
import os
import struct
import threading
import time
from dataclasses import dataclass, field
from typing import Callable, Optional

import torch

from . import _lib
from .checksum import ABS_FLOOR, UNIT_ROUNDOFF, sign_table

# serve.py:55-89: the state row and the capture buffers
STATE_COLS = 4
COL_CHECKS, COL_UNJUDGED = 2, 3
CAPTURE_SLOTS = 4
CAP_REC = 6
CAP_HEAD = 2
CAP_FLAGS = CAP_HEAD + (CAPTURE_SLOTS + 1) * CAP_REC
EPOCH_SHIFT = 32
STEP_MASK = (1 << 32) - 1
OP_SCHEMA = 2

_GOLDEN = 0.5 * (math.sqrt(5.0) - 1.0)


def select_layer(i: int, share: float, offset: int = 0) -> bool:
    """Whether the i-th eligible layer is among a `share` of layers spread evenly by the golden-ratio sequence,
    shifted by `offset` shares (serve.py:104-116: the same selection, so both pick the same layers)."""
    if share >= 1.0:
        return True
    if share <= 0.0:
        return False
    return ((i * _GOLDEN) % 1.0 - offset * share) % 1.0 < share


def _pin_address(t: torch.Tensor) -> None:
    """Tell torch.compile that t keeps its address (buffers the check writes across calls and graph replays)."""
    mark = getattr(getattr(torch, "_dynamo", None), "mark_static_address", None)
    if mark is not None:
        try:
            mark(t)
        except (RuntimeError, TypeError, ValueError):
            pass


def _pattern_pair(width: int, dtype: torch.dtype, dev) -> torch.Tensor:
    """(width, 2): a column of ones and the signed checksum's pattern of that block width, in `dtype`."""
    s = sign_table(dev).view(128, 128)[width - 1, :width]
    return torch.stack([torch.ones_like(s), s], dim=1).to(dtype)


class LayerChecksums:
    """Everything the check needs about one weight matrix W (n outputs x k inputs), computed once on the GPU
    (sdc_layer_constants; the reference builds the same quantities in serve.py:149-211).

    parts      (k, 6nb) view, k-contiguous columns: the three low-precision parts of B2 / scale, B2 the plain and
               signed sums of each block of `block` rows of W (fp32), the layout the check's MFMA kernel reads
    scale, b2n, b2max, bsum        (nb, 2) fp32; bmax, bmax_bias (nb,) fp32; width, wsq (nb,)
    wnorm                          (2, n) fp32: |w_j|_2^2 and |w_j|_1 of every row (the row-block check's A norms)
    pair_full, pair_rem            (bs, 2) / (rem, 2) ones and signs in W's dtype (the op's interface)
    fingerprint                    int64[3] of W's bits (recompute.fingerprint), to notice a rewritten weight
    tensors(with_bias)             the op's arguments after x2 and y2, in the reference's order"""

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor], block: int = 128):
        from .recompute import fingerprint
        W = weight.detach()
        if W.dim() != 2:
            raise ValueError("the serving check takes a 2-D weight (n outputs x k inputs)")
        if W.dtype not in UNIT_ROUNDOFF:
            raise ValueError(f"the serving check takes bf16 and fp16 weights, not {W.dtype}")
        _lib.require_gpu(W)
        if W.stride(1) != 1:
            W = W.contiguous()
        n, k = W.shape
        dt, dev = W.dtype, W.device
        bs = max(1, min(int(block), n))
        self.n, self.k, self.bs, self.dtype = n, k, bs, dt
        self.nbf, self.rem = divmod(n, bs)
        self.nb = nb = self.nbf + (1 if self.rem else 0)
        self.has_bias = bias is not None
        b = None
        if bias is not None:
            b = bias.detach().reshape(-1)
            if b.numel() != n:
                raise ValueError(f"bias of {b.numel()} values for {n} outputs")
            b = b if b.dtype == dt else b.to(dt)
        kp = -(-k // 8) * 8
        L = _lib.lib()
        with torch.no_grad():
            store = torch.empty(6 * nb, kp, dtype=dt, device=dev)
            table = torch.empty(2, nb, 12, dtype=torch.float32, device=dev)
            self.wnorm = torch.empty(2, n, dtype=torch.float32, device=dev)
            ws = _lib.workspace(dev, int(L.sdc_layer_constants_workspace(n, k, bs)))
            rc = L.sdc_layer_constants(_lib.dtype_code(dt), W.data_ptr(), W.stride(0), n, k, bs, _lib.ptr(b),
                                       b.stride(0) if b is not None else 0, sign_table(dev).data_ptr(),
                                       store.data_ptr(), kp, table[0].data_ptr(), table[1].data_ptr(),
                                       self.wnorm.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(W))
            _lib.check(rc, "sdc_layer_constants")
        self.parts = store[:, :k].t()
        cols = table[0]
        self.scale, self.bsum = cols[:, 0:2].contiguous(), cols[:, 2:4].contiguous()
        self.b2n, self.b2max = cols[:, 4:6].contiguous(), cols[:, 6:8].contiguous()
        self.bmax, self.bmax_bias = cols[:, 8].contiguous(), cols[:, 9].contiguous()
        self._nobias = (torch.zeros(nb, device=dev), torch.zeros(nb, 2, device=dev))
        self.width = torch.full((nb,), float(bs), device=dev)
        if self.rem:
            self.width[-1] = float(self.rem)
        self.wsq = self.width.sqrt()
        self.pair_full = _pattern_pair(bs, dt, dev)
        self.pair_rem = _pattern_pair(self.rem, dt, dev) if self.rem else self.pair_full
        self.fingerprint = fingerprint(W)
        # the scoring pass reads one (nb, 12) table per variant: hand the built ones to _packed_consts
        self.bsum._sdc_packed = (table[0], (self.scale.data_ptr(), self.bmax_bias.data_ptr(), self.b2n.data_ptr()))
        self._nobias[1]._sdc_packed = (table[1], (self.scale.data_ptr(), self._nobias[0].data_ptr(),
                                                  self.b2n.data_ptr()))
        for t in self.tensors(True) + self._nobias:
            _pin_address(t)

    def tensors(self, with_bias: bool = True):
        """Arguments of the check op after x2 and y2 (the reference's order, serve.py:239-244)."""
        bmax_bias, bsum = (self.bmax_bias, self.bsum) if with_bias else self._nobias
        return (self.parts, self.pair_full, self.pair_rem, self.scale, self.b2n, self.b2max, self.bmax, bmax_bias,
                bsum, self.wsq, self.width)


def _split3_kmajor(B2: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """(k, c) fp32 -> (k, 3c) parts [hi | mid | lo] in `dt` (checksum._split3), stored as a (3c, k) contiguous
    tensor so every column is k-contiguous."""
    return torch.cat(_parts3(B2.t().contiguous(), dt), dim=0).t()


def _parts3(x: torch.Tensor, dt: torch.dtype):
    hi = x.to(dt)
    r = x - hi
    mid = r.to(dt)
    return hi, mid, (r - mid).to(dt)


def _kmajor_parts(parts: torch.Tensor, scale: torch.Tensor, nb: int, dt: torch.dtype) -> torch.Tensor:
    """`parts` in the kernel's layout: three `dt` parts, k-contiguous.  A LayerChecksums made here already is;
    constants made elsewhere (row-major parts, or fp32 block sums) are converted once and the copy is kept on the
    parts tensor itself, so it lives exactly as long as the constants it copies (keyed by their version, and for
    fp32 block sums by the scale they are divided by)."""
    if parts.shape[1] == 6 * nb and parts.dtype == dt and parts.stride(0) == 1:
        return parts
    fp32_sums = parts.shape[1] == 2 * nb
    key = (parts._version, tuple(parts.shape), parts.dtype, dt,
           (scale.data_ptr(), scale._version) if fp32_sums else None)
    hit = getattr(parts, "_sdc_kmajor", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    with torch.no_grad():
        if parts.shape[1] == 6 * nb and parts.dtype == dt:
            out = parts.t().contiguous().t()
        elif fp32_sums:                                      # plain fp32 B2: split it (scale applies to E after)
            out = _split3_kmajor(parts.float() / scale.reshape(1, 2 * nb), dt)
        else:
            raise ValueError(f"parts of shape {tuple(parts.shape)} don't fit {nb} blocks")
    try:
        parts._sdc_kmajor = (key, out)
    except (AttributeError, RuntimeError):
        pass
    return out


def check_static_impl(x2: torch.Tensor, y2: torch.Tensor, parts: torch.Tensor, pair_full: torch.Tensor,
                      pair_rem: torch.Tensor, scale: torch.Tensor, b2n: torch.Tensor, b2max: torch.Tensor,
                      bmax: torch.Tensor, bmax_bias: torch.Tensor, bsum: torch.Tensor, wsq: torch.Tensor,
                      width: torch.Tensor, state: torch.Tensor, slot: int, z: float, abs_floor: float,
                      cap_meta: Optional[torch.Tensor] = None, cap_data: Optional[torch.Tensor] = None,
                      cap_w: int = 0, cap_tag: int = 0, scores_out: Optional[torch.Tensor] = None,
                      kernel: Optional[str] = None) -> None:
    """Check y2 = x2 @ W^T (+ bias) for one layer on the GPU and fold the worst z into state[slot]; with cap_meta
    and cap_data, keep the row that alarmed (serve.py:257-270).  No host sync.  scores_out (tests): a (m, nb, 2)
    fp32 tensor that receives every checksum's score; kernel ("v1" | "v3") forces one design."""
    m, n = y2.shape
    if m == 0 or n == 0:
        return
    _lib.require_gpu(x2, y2, parts, state)
    dt = y2.dtype
    if x2.dtype != dt:
        x2 = x2.to(dt)
    k = x2.shape[1]
    nb = b2n.shape[0]
    bs = pair_full.shape[0]
    if bs > 128:
        raise _lib.HipLibraryError(f"the serving check takes blocks up to 128 wide, not {bs}")
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    P = _kmajor_parts(parts, scale, nb, dt)
    counts = 1 if (state.dim() == 2 and state.shape[1] >= STATE_COLS) else 0
    capture = cap_meta is not None and cap_data is not None
    if capture and not (cap_meta.dtype == torch.int64 and cap_data.dtype == torch.float32 and cap_w >= bs
                        and cap_data.shape[1] >= cap_w + k and cap_meta.numel() > CAP_FLAGS + slot):
        raise ValueError("the capture buffer doesn't fit this layer")
    for t in (scale, b2n, b2max, bmax, bmax_bias, bsum):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("layer constants must be contiguous fp32 tensors")
    L = _lib.lib()
    # the parts in fragment order for the tall-tile GEMM (made once, kept on the parts tensor), where it applies
    frag = None
    if k % 512 == 0 and x2.stride(1) == 1 and x2.data_ptr() % 16 == 0 and (x2.stride(0) * x2.element_size()) % 16 == 0:
        from .linear import _fragments
        frag = _fragments(P, 2 * nb, k)
    ws_bytes = int(L.sdc_check_static_workspace(m, k, n, bs))
    ws = _lib.workspace(y2.device, ws_bytes)
    row = state.data_ptr() + slot * state.stride(0) * state.element_size()
    rc = L.sdc_check_static(
        _lib.dtype_code(dt), x2.data_ptr(), x2.stride(0), x2.stride(1), y2.data_ptr(), y2.stride(0), y2.stride(1),
        m, k, n, bs, P.data_ptr(), P.stride(0), P.stride(1), 3, sign_table(y2.device).data_ptr(),
        scale.data_ptr(), b2n.data_ptr(), b2max.data_ptr(), bmax.data_ptr(), bmax_bias.data_ptr(), bsum.data_ptr(),
        row, counts, int(slot), float(z), float(abs_floor),
        cap_meta.data_ptr() if capture else None, cap_data.data_ptr() if capture else None,
        cap_data.stride(0) if capture else 0, int(cap_w), int(cap_tag), CAP_FLAGS, CAPTURE_SLOTS,
        ws.data_ptr(), ws_bytes, None if scores_out is None else scores_out.data_ptr(),
        kernel_mode() if kernel is None else {"v1": 1, "v3": 3, "v3-serial": 4}[kernel],
        _packed_consts(scale, b2n, b2max, bmax, bmax_bias, bsum).data_ptr(), _lib.ptr(frag), _lib.stream_of(y2))
    _lib.check(rc, "sdc_check_static")


def _packed_consts(scale, b2n, b2max, bmax, bmax_bias, bsum) -> torch.Tensor:
    """The per-block constants as one (nb, 12) fp32 table (three 16-byte loads per block in the kernel):
    [scale, bsum, b2n, b2max, bmax, bmax_bias, 0, 0].  Kept on the bsum tensor object (with and without the
    bias, LayerChecksums hands different bsum tensors), so it lives exactly as long as the constants it packs."""
    packed = getattr(bsum, "_sdc_packed", None)
    if packed is not None and packed[1] == (scale.data_ptr(), bmax_bias.data_ptr(), b2n.data_ptr()):
        return packed[0]
    nb = b2n.shape[0]
    z = torch.zeros(nb, 2, dtype=torch.float32, device=bsum.device)
    t = torch.cat([scale.view(nb, 2), bsum.view(nb, 2), b2n.view(nb, 2), b2max.view(nb, 2),
                   torch.stack([bmax.view(nb), bmax_bias.view(nb)], 1), z], dim=1).contiguous()
    try:
        bsum._sdc_packed = (t, (scale.data_ptr(), bmax_bias.data_ptr(), b2n.data_ptr()))
    except (AttributeError, RuntimeError):
        pass
    return t


def kernel_mode() -> int:
    """0: the design by batch size; SDCGUARD_SERVE_KERNEL=v1|v3 forces one (_serve_fast.py:600-606)."""
    v = os.environ.get("SDCGUARD_SERVE_KERNEL", "auto")
    return {"v1": 1, "v3": 3}.get(v, 0)


# the reference routes between its Triton and PyTorch checks here; this build has one implementation
check_static_any = check_static_impl


def decode_state(rows: torch.Tensor):
    """(z, flat index, noise) of every state row (the reference's decode_state, serve.py:399-404)."""
    return [decode(a, b) for a, b in rows[:, :2].detach().to("cpu").tolist()]


def decode_counts(rows: torch.Tensor):
    """(checks executed, unjudged checksums) of every state row (serve.py:407-412); zeros for rows without them."""
    if rows.dim() != 2 or rows.shape[1] < STATE_COLS:
        return [(0, 0) for _ in range(rows.shape[0])]
    return [(int(r[COL_CHECKS]), int(r[COL_UNJUDGED])) for r in rows.detach().to("cpu").tolist()]


def decode(key_i: int, key_d: int, *counts: int):
    """(z, flat position, noise) from a state row (_serve_fast.py:673-679)."""
    zb = (int(key_i) >> 32) & 0xFFFFFFFF
    z = struct.unpack("<f", struct.pack("<I", zb))[0]
    nz = struct.unpack("<f", struct.pack("<I", int(key_d) & 0xFFFFFFFF))[0]
    return z, int(key_i) & 0xFFFFFFFF, nz


_lib_lock = threading.Lock()
_OP = [None]


def _op():
    """sdcguard::check_static, registered once with the reference's argument list (serve.py:465-489)."""
    with _lib_lock:
        if _OP[0] is None:
            try:
                @torch.library.custom_op("sdcguard::check_static", mutates_args=("state", "cap_meta", "cap_data"))
                def check_static(x2: torch.Tensor, y2: torch.Tensor, parts: torch.Tensor, pair_full: torch.Tensor,
                                 pair_rem: torch.Tensor, scale: torch.Tensor, b2n: torch.Tensor, b2max: torch.Tensor,
                                 bmax: torch.Tensor, bmax_bias: torch.Tensor, bsum: torch.Tensor, wsq: torch.Tensor,
                                 width: torch.Tensor, state: torch.Tensor, slot: int, z: float, abs_floor: float,
                                 cap_meta: torch.Tensor, cap_data: torch.Tensor, cap_w: int, cap_tag: int) -> None:
                    check_static_impl(x2, y2, parts, pair_full, pair_rem, scale, b2n, b2max, bmax, bmax_bias, bsum,
                                      wsq, width, state, slot, z, abs_floor, cap_meta, cap_data, cap_w, cap_tag)

                @check_static.register_fake
                def _(x2, y2, parts, pair_full, pair_rem, scale, b2n, b2max, bmax, bmax_bias, bsum, wsq, width, state,
                      slot, z, abs_floor, cap_meta, cap_data, cap_w, cap_tag):
                    return None

                _OP[0] = torch.ops.sdcguard.check_static
            except (AttributeError, RuntimeError):
                _OP[0] = getattr(getattr(torch.ops, "sdcguard", None), "check_static", None) or check_static_impl
        return _OP[0]


@dataclass
class SDCEvent:
    """One alert (the fields of the reference's events.SDCEvent that the serving check fills)."""
    detector: str
    layer: str
    z: float
    row: Optional[int] = None
    col_block: Optional[int] = None
    noise: Optional[float] = None
    nonfinite: bool = False
    time: float = field(default_factory=time.time)
    extra: dict = field(default_factory=dict)


class _DeviceRows:
    """What a guard keeps on one device: the int64 state rows of its layers, the capture area (flags and the rows
    kept for a recheck), and the snapshot of the state on its way to the host."""

    def __init__(self, device: torch.device, rows: int, kmax: int, cap_w: int):
        self.device = device
        self.state = torch.zeros(rows, STATE_COLS, dtype=torch.int64, device=device)
        self.cap_meta = torch.zeros(CAP_FLAGS + rows, dtype=torch.int64, device=device)
        self.cap_data = torch.zeros(CAPTURE_SLOTS + 1, cap_w + kmax, dtype=torch.float32, device=device)
        self.in_flight = None            # (pinned host copy, event recorded after the copy)
        self.epoch = 0
        for t in (self.state, self.cap_meta, self.cap_data):
            _pin_address(t)

    def fits(self, rows: int, kmax: int, cap_w: int) -> bool:
        return self.state.shape[0] >= rows and self.cap_data.shape[1] >= cap_w + kmax

    def enlarged(self, rows: int, kmax: int, cap_w: int) -> "_DeviceRows":
        """A bigger copy (room for twice the layers, depth rounded up to 1024) keeping what this one holds."""
        new = _DeviceRows(self.device, max(rows, 2 * self.state.shape[0]), -(-max(kmax, 1) // 1024) * 1024, cap_w)
        new.state[:self.state.shape[0]] = self.state
        new.cap_meta[:CAP_FLAGS + self.state.shape[0]] = self.cap_meta
        new.cap_data[:, :self.cap_data.shape[1]] = self.cap_data
        new.epoch = self.epoch
        return new

    def take(self, n: int, wait: bool):
        """Start copying the first n state rows to the host, then clear them and open a new capture epoch, in stream
        order on the current stream.  wait: return the host rows; else return None and keep them in flight."""
        stream = torch.cuda.current_stream(self.device)
        if wait:
            host = self.state[:n].to("cpu")
        else:
            host = torch.empty((n, STATE_COLS), dtype=torch.int64, pin_memory=True)
            host.copy_(self.state[:n], non_blocking=True)
        self.state[:n].zero_()
        self.epoch += 1
        self.cap_meta[1:2].add_(1 << EPOCH_SHIFT)
        self.cap_meta[CAP_FLAGS:CAP_FLAGS + n].zero_()
        if wait:
            return host
        ev = torch.cuda.Event()
        ev.record(stream)
        self.in_flight = (host, ev)
        return None

    def landed(self, block: bool):
        """The host rows of the snapshot in flight once they have arrived (block: wait for them), else None."""
        if self.in_flight is None:
            return None
        host, ev = self.in_flight
        if block:
            ev.synchronize()
        elif not ev.query():
            return None
        self.in_flight = None
        return host


class ServeGuard:
    """Always-on checks for inference (the reference's serve.ServeGuard, serve.py:548-1170, for its checksum leg).

    attach(model) checks every bf16/fp16 nn.Linear through a forward hook (the layer's own forward runs unchanged);
    poll() reads the per-layer worst scores back without stalling the GPU and returns the alerts; detach() removes
    the hooks.  check(slot, x, y) / op_args(slot) serve callers that run the layer themselves (a vLLM linear
    method)."""

    def __init__(self, z: float = 6.0, block: int = 128, abs_floor: float = ABS_FLOOR,
                 on_alert: Optional[Callable[[SDCEvent], None]] = None):
        z = float(z)
        if not 0 < z < math.inf:
            raise ValueError(f"z must be a positive number (the alert line in noise units), not {z!r}")
        if not 1 <= int(block) <= 128:
            raise ValueError("blocks are 1 to 128 outputs wide")
        self.z, self.block, self.abs_floor = z, int(block), abs_floor
        self.on_alert = on_alert
        self.enabled = True
        self.layers: list = []                 # per slot: name, module, cs, device, hook handle
        self._rows: dict = {}                  # device -> _DeviceRows
        self._cap_w = max(128, int(block))
        self.worst_seen: dict = {}
        self.checks_seen: dict = {}
        self.unjudged_seen: dict = {}
        self.events: list = []
        self.unsupported: dict = {}
        self._scan = None                      # the weight scan (weight_scan())
        self._fp8 = None                       # FP8 quantization checks (fp8_checks())
        self._moe = None                       # fused MoE checks (moe_checks())
        self._attn = None                      # sampled attention recompute (attn_checks())
        self._route = None                     # MoE router checks (route_checks())
        self._marked_step: Optional[int] = None
        self.stats = {"layers": 0, "skipped_layers": 0, "polls": 0, "alerts": 0, "checks_executed": 0,
                      "unjudged_checksums": 0}

    # ---------------------------------------------------------------- layers
    @staticmethod
    def _why_not(mod: torch.nn.Module) -> Optional[str]:
        if getattr(mod, "_sdcguard_slot", None):
            return "already checked by another ServeGuard"
        w = getattr(mod, "weight", None)
        if not torch.is_tensor(w) or w.dtype not in UNIT_ROUNDOFF or w.numel() == 0:
            return f"{getattr(w, 'dtype', None)} weights or no weights: not checked"
        if not w.is_cuda:
            return "weights not on a GPU: not checked"
        if "forward" in mod.__dict__ or type(mod).forward is not torch.nn.Linear.forward:
            return "forward replaced: its output need not be x W^T + b, not checked"
        return None

    def attach(self, model: torch.nn.Module, share: float = 1.0, offset: int = 0) -> "ServeGuard":
        """Check every eligible nn.Linear of `model` (a golden-ratio spread `share` of them)."""
        eligible = 0
        for name, mod in model.named_modules():
            if not isinstance(mod, torch.nn.Linear):
                continue
            label = name or type(mod).__name__
            why = self._why_not(mod)
            if why is not None:
                self.unsupported[label] = why
                self.stats["skipped_layers"] += why != "already checked by another ServeGuard"
                continue
            chosen = select_layer(eligible, share, offset)
            eligible += 1
            if not chosen:
                self.stats["skipped_layers"] += 1
                continue
            slot = self.add_layer(mod, label)
            self.layers[slot]["hook"] = mod.register_forward_hook(self._hook(slot))
        return self

    def add_layer(self, mod: torch.nn.Module, name: str, weight: Optional[torch.Tensor] = None,
                  bias: Optional[torch.Tensor] = None) -> int:
        """Register a layer (its constants are built now) and return its slot; no hook is installed."""
        w = mod.weight if weight is None else weight
        b = getattr(mod, "bias", None) if bias is None else bias
        with torch.inference_mode(False), torch.no_grad():
            cs = LayerChecksums(w, b, self.block)
        slot = len(self.layers)
        taken = {lay["name"] for lay in self.layers}
        if not name or name in taken:
            name = f"{name or type(mod).__name__}#{slot + 1}"
        self.layers.append({"name": name, "module": mod, "cs": cs, "device": w.device, "hook": None})
        mod._sdcguard_slot = slot + 1
        mod._sdcguard_name = name
        kmax = max(lay["cs"].k for lay in self.layers if lay["device"] == w.device)
        rows = self._rows.get(w.device)
        if rows is None:
            self._rows[w.device] = _DeviceRows(w.device, 4096, -(-max(kmax, 8192) // 1024) * 1024, self._cap_w)
        elif not rows.fits(slot + 1, kmax, self._cap_w):
            self._rows[w.device] = rows.enlarged(slot + 1, kmax, self._cap_w)
        self.stats["layers"] += 1
        return slot

    def replace_layer(self, slot: int, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> int:
        """New constants for layer `slot` after its weights were reloaded; the slot and its state row stay."""
        lay = self.layers[slot]
        with torch.inference_mode(False), torch.no_grad():
            lay["cs"] = LayerChecksums(weight, bias, self.block)
        rows = self._rows[lay["device"]]
        kmax = max(x["cs"].k for x in self.layers if x["device"] == lay["device"])
        if not rows.fits(len(self.layers), kmax, self._cap_w):
            self._rows[lay["device"]] = rows.enlarged(len(self.layers), kmax, self._cap_w)
        return slot

    def _hook(self, slot: int):
        cs = self.layers[slot]["cs"]

        def after_forward(mod, args, out):
            if not self.enabled or not args or not torch.is_tensor(out) or out.dtype != cs.dtype:
                return None
            x = args[0]
            if not torch.is_tensor(x) or x.numel() == 0 or x.shape[-1] != cs.k or out.shape[-1] != cs.n:
                return None
            run = _op() if torch.compiler.is_compiling() else check_static_impl
            run(x.reshape(-1, cs.k), out.reshape(-1, cs.n), *self.op_args(slot, True))
            return None

        return after_forward

    def state(self, device) -> torch.Tensor:
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        return self._rows[device].state

    def op_args(self, slot: int, with_bias: bool = True) -> tuple:
        """The op's arguments after x2 and y2 for layer `slot` (constants, state, slot, z, floor, capture area)."""
        lay = self.layers[slot]
        r = self._rows[lay["device"]]
        tag = 2 * (slot + 1) + int(with_bias and lay["cs"].has_bias)
        return (*lay["cs"].tensors(with_bias), r.state, slot, self.z, float(self.abs_floor), r.cap_meta, r.cap_data,
                self._cap_w, tag)

    def check(self, slot: int, x: torch.Tensor, y: torch.Tensor, with_bias: bool = True) -> None:
        """Queue the check of layer `slot` for its input x and output y (any leading dims); no host sync."""
        cs = self.layers[slot]["cs"]
        if not self.enabled or y.dtype not in UNIT_ROUNDOFF or x.shape[-1] != cs.k or y.shape[-1] != cs.n:
            return
        check_static_impl(x.reshape(-1, cs.k), y.reshape(-1, cs.n), *self.op_args(slot, with_bias))

    def read_slot(self, slot: int):
        """(z, flat index, noise) of one layer's state row now (waits for the GPU)."""
        lay = self.layers[slot]
        return decode_state(self._rows[lay["device"]].state[slot:slot + 1])[0]

    def verify_weights(self) -> list:
        """Names of the layers whose weights no longer hold the bits their constants were built from."""
        from .recompute import fingerprint
        return [lay["name"] for lay in self.layers
                if not torch.equal(fingerprint(lay["module"].weight), lay["cs"].fingerprint)]

    # ---------------------------------------------------------------- results
    def poll(self, wait: bool = False) -> list:
        """Alerts since the last poll.  Without wait it never stalls the host: it reports the snapshot started by
        the previous poll once that has arrived and starts the next one."""
        self.stats["polls"] += 1
        n = len(self.layers)
        events = []
        for dev, rows in self._rows.items():
            done = rows.landed(block=wait)
            if done is not None:
                events += self._report(dev, done)
            if wait:
                events += self._report(dev, rows.take(n, wait=True))
            elif rows.in_flight is None:
                rows.take(n, wait=False)
        if self._fp8 is not None:
            events += self._fp8.poll(wait)
        if self._moe is not None and self._moe.finalized:
            events += self._moe.poll(wait)
        if self._attn is not None and self._attn.finalized:
            events += self._attn.poll(wait)
        if self._route is not None and self._route.finalized:
            events += self._route.poll(wait)
        if self._scan is not None:
            events += self._scan.poll(wait)
        return events

    def fp8_checks(self):
        """The FP8 input-quantization checks of this guard's FP8 layers (serve_fp8.Fp8Checks), created on first use;
        mark_step / end_step / poll reach them through the guard."""
        if self._fp8 is None:
            from .serve_fp8 import Fp8Checks
            self._fp8 = Fp8Checks(self)
        return self._fp8

    def moe_checks(self, line: Optional[float] = None):
        """The sampled recompute checks of fused MoE layers (serve_moe.MoEChecks), created on first use: add() the
        layers, finalize() before capture; mark_step / end_step / poll reach them through the guard."""
        if self._moe is None:
            from .serve_moe import MOE_Z, MoEChecks
            self._moe = MoEChecks(self, MOE_Z if line is None else line)
        return self._moe

    def attn_checks(self, line: Optional[float] = None):
        """The sampled attention recompute of the serving stack's attention layers (serve_attn.AttnChecks), created
        on first use: add() the layers, finalize() before capture; mark_step / end_step / poll reach it through the
        guard."""
        if self._attn is None:
            from .serve_attn import ATTN_Z, AttnChecks
            self._attn = AttnChecks(self, ATTN_Z if line is None else line)
        return self._attn

    def route_checks(self):
        """The MoE router checks (serve_route.RouteChecks), created on first use: add() the routers, finalize()
        before capture; mark_step / end_step / poll reach them through the guard."""
        if self._route is None:
            from .serve_route import RouteChecks
            self._route = RouteChecks(self)
        return self._route

    def _step_checks(self) -> list:
        return [c for c in (self._fp8, self._moe, self._attn, self._route) if c is not None]

    def end_step(self) -> None:
        """After a model step's work is queued (the per-step checks stop judging until the next mark_step)."""
        for c in self._step_checks():
            c.end_step()

    def weight_scan(self, budget_mb: Optional[float] = None, **kw):
        """The scheduled weight scan of this guard's layers (serve_weights.WeightScan), created on the first call:
        each poll() fingerprints the next layers' tensors, up to budget_mb, and compares them with their references."""
        if self._scan is None:
            from .serve_weights import DEFAULT_BUDGET_MB, WeightScan
            self._scan = WeightScan(self, DEFAULT_BUDGET_MB if budget_mb is None else budget_mb, **kw)
            self._scan.sync()
        return self._scan

    def mark_step(self, step: int, rows: Optional[int] = None) -> None:
        """Stamp the capture area with the serving step (kept rows carry it)."""
        self._marked_step = int(step)
        for c in self._step_checks():
            c.mark_step(step, rows)
        step = int(step) & STEP_MASK
        for r in self._rows.values():
            r.cap_meta[1:2].fill_((r.epoch << EPOCH_SHIFT) | step)

    def _report(self, dev, host: torch.Tensor) -> list:
        out = []
        keys = decode_state(host)
        counts = decode_counts(host)
        for slot, lay in enumerate(self.layers):
            if lay["device"] != dev or slot >= host.shape[0]:
                continue
            name, cs = lay["name"], lay["cs"]
            z, flat, noise = keys[slot]
            checks, unjudged = counts[slot]
            self.checks_seen[name] = self.checks_seen.get(name, 0) + checks
            self.unjudged_seen[name] = self.unjudged_seen.get(name, 0) + unjudged
            self.stats["checks_executed"] += checks
            self.stats["unjudged_checksums"] += unjudged
            self.worst_seen[name] = max(self.worst_seen.get(name, 0.0), z)
            if not z > self.z:
                continue
            blk = flat >> 1
            ev = SDCEvent(detector="serve_checksum", layer=name, z=z, row=blk // cs.nb, col_block=blk % cs.nb,
                          noise=noise, nonfinite=not math.isfinite(z) or noise != noise,
                          extra={"checksum": "signed" if flat & 1 else "plain"})
            out.append(ev)
            self.events.append(ev)
            self.stats["alerts"] += 1
            if self.on_alert is not None:
                self.on_alert(ev)
        return out

    def captured(self, dev) -> list:
        """(record, y block, x row) of every row kept on a device in the current epoch (waits for the GPU)."""
        r = self._rows[torch.device(dev)]
        meta = r.cap_meta[:CAP_FLAGS].to("cpu")
        kept = min(int(meta[0]), CAPTURE_SLOTS)
        recs = meta[CAP_HEAD:CAP_HEAD + kept * CAP_REC].view(kept, CAP_REC).tolist()
        data = r.cap_data[:kept].to("cpu")
        out = []
        for i, rec in enumerate(recs):
            cs = self.layers[rec[0] // 2 - 1]["cs"]
            width = cs.bs if rec[2] < cs.nbf else cs.rem
            out.append((rec, data[i, :width], data[i, self._cap_w:self._cap_w + cs.k]))
        return out

    def detach(self) -> None:
        """Final poll (waits), then remove the hooks and forget the layers."""
        try:
            if self.layers:
                self.poll(wait=True)
        finally:
            for lay in self.layers:
                if lay.get("hook") is not None:
                    lay["hook"].remove()
                for attr in ("_sdcguard_slot", "_sdcguard_name"):
                    lay["module"].__dict__.pop(attr, None)
            for sub in self._step_checks():
                sub.detach()
            self._fp8 = self._moe = self._attn = self._route = None
            self.layers.clear()
            self._rows.clear()
            self._scan = None
            self.stats["layers"] = 0
