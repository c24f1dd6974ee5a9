"""Serving check: every bf16/fp16 linear layer on every forward pass (reference: serve.py).

Weights do not change while a model serves, so each layer's block sums are computed once (LayerChecksums) and
every forward pass only reads the layer's input x and output y again:

    expected = x @ (block sums of W)       MFMA, three low-precision parts of the fp32 sums
    actual   = block sums of y             one pass over y
    z        = |expected - actual| / rounding noise,  fault above z (default 6)

The work runs in libsdcguard_hip.so (sdc_check_static), two launches per layer, no host synchronisation; the
worst score goes into a per-layer int64 state row with atomic maxima and is read back asynchronously by
ServeGuard.poll().  The custom op sdcguard::check_static keeps the reference's argument list (serve.py:465-489),
so torch.compile sees one opaque call and HIP graphs capture its kernels.
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
from .checksum import ABS_FLOOR, UNIT_ROUNDOFF, _signs, sign_table

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

_PHI = (math.sqrt(5.0) - 1.0) / 2.0


def select_layer(i: int, share: float, offset: int = 0) -> bool:
    """Golden-ratio spread of a checked share of layers (serve.py:104-116)."""
    if share >= 1.0:
        return True
    if share <= 0.0:
        return False
    return ((i * _PHI) % 1.0 - offset * share) % 1.0 < share


def _static(t: torch.Tensor) -> None:
    try:
        torch._dynamo.mark_static_address(t)
    except Exception:  # noqa: BLE001
        pass


class LayerChecksums:
    """Everything the check needs about one weight matrix W (n outputs x k inputs), computed once
    (serve.py:140-244).  `parts` is the (k x 6nb) matrix of the three low-precision parts of B2 / scale, stored
    k-contiguous per column (a transposed view of a (6nb x k) tensor): the layout the MFMA kernel reads."""

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor], block: int = 128):
        with torch.autocast(device_type=weight.device.type, enabled=False), torch.no_grad():
            self._initialize(weight, bias, block)

    def _initialize(self, weight: torch.Tensor, bias: Optional[torch.Tensor], block: int) -> None:
        W = weight.detach()
        n, k = W.shape
        dt, dev = W.dtype, W.device
        if dt not in UNIT_ROUNDOFF:
            raise ValueError(f"the serving check takes bf16 and fp16 weights, not {dt}")
        bs = max(1, min(block, n))
        nbf, rem = n // bs, n % bs
        nb = nbf + (1 if rem else 0)
        self.n, self.k, self.nb, self.bs, self.nbf, self.rem, self.dtype = n, k, nb, bs, nbf, rem, dt
        self.has_bias = bias is not None
        self.pair_full = self._pair(bs, dt, dev)
        self.pair_rem = self._pair(rem, dt, dev) if rem else self.pair_full
        Wf = W.float()
        cols = []
        if nbf:
            Wb = Wf[:nbf * bs].view(nbf, bs, k)
            cols.append(torch.einsum("bjk,jc->kbc", Wb, self._pair(bs, torch.float32, dev)).reshape(k, 2 * nbf))
        if rem:
            cols.append(torch.einsum("jk,jc->kc", Wf[nbf * bs:], self._pair(rem, torch.float32, dev)))
        B2 = torch.cat(cols, dim=1).contiguous()                                # (k, 2nb) fp32
        del Wf
        self.b2n = torch.linalg.vector_norm(B2, dim=0).view(nb, 2)
        self.b2max = torch.linalg.vector_norm(B2, ord=float("inf"), dim=0).view(nb, 2)
        if dt == torch.float16:
            amax = B2.abs().amax(dim=0)
            ok = torch.isfinite(amax) & (amax > 0)
            scale = torch.where(ok, torch.exp2(torch.ceil(torch.log2(amax.clamp_min(1e-30)))), 1.0)
        else:
            scale = torch.ones(2 * nb, device=dev, dtype=torch.float32)
        self.scale = scale.view(nb, 2)
        # (6nb, k) contiguous: part p of column c is row p * 2nb + c; `parts` is its (k, 6nb) transpose
        self.parts = _split3_kmajor(B2 / scale, dt)
        rows_max = W.float().abs().amax(dim=1)
        self.bmax = self._block_reduce(rows_max, nbf, bs, rem)
        if bias is not None:
            bf = bias.detach().float()
            bp = []
            if nbf:
                bp.append(bf[:nbf * bs].view(nbf, bs) @ self._pair(bs, torch.float32, dev))
            if rem:
                bp.append((bf[nbf * bs:] @ self._pair(rem, torch.float32, dev)).view(1, 2))
            self.bsum = torch.cat(bp, dim=0)
            self.bmax_bias = self._block_reduce(bf.abs(), nbf, bs, rem)
        else:
            self.bsum = torch.zeros(nb, 2, device=dev, dtype=torch.float32)
            self.bmax_bias = torch.zeros(nb, device=dev, dtype=torch.float32)
        self._z1 = torch.zeros(nb, device=dev, dtype=torch.float32)
        self._z2 = torch.zeros(nb, 2, device=dev, dtype=torch.float32)
        width = torch.full((nb,), float(bs), device=dev, dtype=torch.float32)
        if rem:
            width[-1] = float(rem)
        self.width = width
        self.wsq = width.sqrt()
        self.fingerprint = self._fingerprint(W)
        for wb in (True, False):
            _packed_consts(*(self.tensors(wb)[i] for i in (3, 4, 5, 6, 7, 8)))
        for t in self.tensors(True) + self.tensors(False):
            _static(t)

    @staticmethod
    def _pair(width: int, dtype: torch.dtype, dev) -> torch.Tensor:
        s = _signs(width, dev)
        return torch.stack([torch.ones_like(s), s], dim=1).to(dtype)

    @staticmethod
    def _block_reduce(v: torch.Tensor, nbf: int, bs: int, rem: int) -> torch.Tensor:
        out = []
        if nbf:
            out.append(v[:nbf * bs].view(nbf, bs).amax(dim=1))
        if rem:
            out.append(v[nbf * bs:].amax().view(1))
        return torch.cat(out)

    @staticmethod
    def _fingerprint(W: torch.Tensor) -> torch.Tensor:
        """serve.py:226-237: sums of the weights' raw bits, plain and weighted by position mod 65521."""
        bits = W.contiguous().view(-1).view(torch.int16 if W.element_size() == 2 else torch.int32)
        tot = torch.zeros(2, dtype=torch.int64, device=W.device)
        chunk = 1 << 24
        for i in range(0, bits.numel(), chunk):
            b = bits[i:i + chunk].to(torch.int64)
            pos = torch.arange(i, i + b.numel(), device=W.device, dtype=torch.int64) % 65521 + 1
            tot += torch.stack([b.sum(), (b * pos).sum()])
        return tot

    def tensors(self, with_bias: bool = True):
        """Arguments of the check op after x2 and y2 (serve.py:239-244)."""
        bmb, bs = (self.bmax_bias, self.bsum) if with_bias else (self._z1, self._z2)
        return (self.parts, self.pair_full, self.pair_rem, self.scale, self.b2n, self.b2max, self.bmax, bmb, bs,
                self.wsq, self.width)


def _split3_kmajor(B2: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """(k, c) fp32 -> (k, 3c) parts [hi | mid | lo] in `dt` (checksum._split3), stored as a (3c, k) contiguous
    tensor so every column is k-contiguous."""
    return torch.cat(_parts3(B2.t().contiguous(), dt), dim=0).t()


def _parts3(x: torch.Tensor, dt: torch.dtype):
    hi = x.to(dt)
    r = x - hi
    mid = r.to(dt)
    return hi, mid, (r - mid).to(dt)


_KMAJOR: dict = {}
_KMAJOR_LOCK = threading.Lock()


def _kmajor_parts(parts: torch.Tensor, scale: torch.Tensor, nb: int, dt: torch.dtype) -> torch.Tensor:
    """`parts` in the kernel's layout: three `dt` parts, k-contiguous.  A LayerChecksums made here already is;
    constants made elsewhere (row-major parts, or fp32 block sums) are converted once and kept."""
    if parts.shape[1] == 6 * nb and parts.dtype == dt and parts.stride(0) == 1:
        return parts
    key = (parts.data_ptr(), parts._version, tuple(parts.shape), parts.dtype, str(parts.device))
    hit = _KMAJOR.get(key)
    if hit is not None:
        return hit
    with torch.no_grad():
        if parts.shape[1] == 6 * nb and parts.dtype == dt:
            out = parts.t().contiguous().t()
        elif parts.shape[1] == 2 * nb:                       # plain fp32 B2: split it (scale applies to E after)
            out = _split3_kmajor(parts.float() / scale.reshape(1, 2 * nb), dt)
        else:
            raise ValueError(f"parts of shape {tuple(parts.shape)} don't fit {nb} blocks")
    with _KMAJOR_LOCK:
        if len(_KMAJOR) > 64:
            _KMAJOR.clear()
        _KMAJOR[key] = out
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
        _packed_consts(scale, b2n, b2max, bmax, bmax_bias, bsum).data_ptr(), _lib.stream_of(y2))
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
    """(z, flat index, noise) per row of a state tensor on the CPU (serve.py:399-404)."""
    zs = (rows[:, 0] >> 32).to(torch.int32).view(torch.float32).tolist()
    flats = (rows[:, 0] & 0xFFFFFFFF).tolist()
    nzs = (rows[:, 1] & 0xFFFFFFFF).to(torch.int32).view(torch.float32).tolist()
    return list(zip(zs, flats, nzs))


def decode_counts(rows: torch.Tensor):
    """(checks executed, unjudged checksums) per row (serve.py:407-412)."""
    if rows.dim() != 2 or rows.shape[1] < STATE_COLS:
        return [(0, 0)] * rows.shape[0]
    return list(zip(rows[:, COL_CHECKS].tolist(), rows[:, COL_UNJUDGED].tolist()))


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


class ServeGuard:
    """Always-on checks for inference (serve.py:548-).  attach(model) checks every bf16/fp16 nn.Linear; poll()
    reads the per-layer state back (asynchronously unless wait=True) and returns alerts."""

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
        self.layers: list = []
        self._state: dict = {}
        self._cap: dict = {}
        self._cap_w = max(128, int(block))
        self._host: dict = {}
        self._epoch: dict = {}
        self.worst_seen: dict = {}
        self.checks_seen: dict = {}
        self.unjudged_seen: dict = {}
        self.events: list = []
        self.unsupported: dict = {}
        self.stats = {"layers": 0, "skipped_layers": 0, "polls": 0, "alerts": 0, "checks_executed": 0,
                      "unjudged_checksums": 0}

    # ---------------------------------------------------------------- setup
    def attach(self, model: torch.nn.Module, share: float = 1.0, offset: int = 0) -> "ServeGuard":
        i = 0
        for name, mod in model.named_modules():
            if not isinstance(mod, torch.nn.Linear):
                continue
            label = name or type(mod).__name__
            if getattr(mod, "_sdcguard_slot", None):
                self.unsupported[label] = "already checked by another ServeGuard"
                continue
            if mod.weight.dtype not in UNIT_ROUNDOFF or mod.weight.numel() == 0:
                self.unsupported[label] = f"{mod.weight.dtype} weights or no weights: not checked"
                self.stats["skipped_layers"] += 1
                continue
            if type(mod).forward is not torch.nn.Linear.forward or "forward" in mod.__dict__:
                self.unsupported[label] = "forward replaced: not checked"
                self.stats["skipped_layers"] += 1
                continue
            take = select_layer(i, share, offset)
            i += 1
            if not take:
                self.stats["skipped_layers"] += 1
                continue
            slot = self.add_layer(mod, label)
            mod.forward = self._make_forward(mod)
            self.layers[slot]["took_over"] = True
        return self

    def add_layer(self, mod: torch.nn.Module, name: str, weight: Optional[torch.Tensor] = None,
                  bias: Optional[torch.Tensor] = None) -> int:
        w = mod.weight if weight is None else weight
        b = getattr(mod, "bias", None) if bias is None else bias
        with torch.inference_mode(False), torch.no_grad():
            cs = LayerChecksums(w, b, self.block)
            slot = len(self.layers)
            if not name or any(lay["name"] == name for lay in self.layers):
                name = f"{name or type(mod).__name__}#{slot + 1}"
            self.layers.append({"name": name, "module": mod, "cs": cs, "device": w.device})
            mod._sdcguard_slot = slot + 1
            mod._sdcguard_name = name
            self._grow(w.device)
        self.stats["layers"] += 1
        return slot

    def _grow(self, device: torch.device) -> None:
        n = len(self.layers)
        kmax = max([lay["cs"].k for lay in self.layers if lay["device"] == device] or [1])
        st = self._state.get(device)
        if st is None or st.shape[0] < n:
            new = torch.zeros(max(4096, 2 * n), STATE_COLS, device=device, dtype=torch.int64)
            if st is not None:
                new[:st.shape[0]] = st
            _static(new)
            self._state[device] = new
        st = self._state[device]
        cm, cd = self._cap.get(device, (None, None))
        if cm is None or cm.numel() < CAP_FLAGS + st.shape[0]:
            new = torch.zeros(CAP_FLAGS + st.shape[0], device=device, dtype=torch.int64)
            if cm is not None:
                new[:cm.numel()] = cm
            cm = new
        if cd is None or cd.shape[1] < self._cap_w + kmax:
            new = torch.zeros(CAPTURE_SLOTS + 1, self._cap_w + max(8192, -(-kmax // 1024) * 1024), device=device,
                              dtype=torch.float32)
            if cd is not None:
                new[:, :cd.shape[1]] = cd
            cd = new
        self._cap[device] = (cm, cd)

    def state(self, device) -> torch.Tensor:
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        return self._state[device]

    def op_args(self, slot: int, with_bias: bool = True) -> tuple:
        lay = self.layers[slot]
        cm, cd = self._cap[lay["device"]]
        tag = (slot + 1) * 2 + (1 if with_bias and lay["cs"].has_bias else 0)
        return (*lay["cs"].tensors(with_bias), self._state[lay["device"]], slot, float(self.z), float(self.abs_floor),
                cm, cd, self._cap_w, tag)

    def check(self, slot: int, x: torch.Tensor, y: torch.Tensor, with_bias: bool = True) -> None:
        """Queue the check of layer `slot` for input x and output y (any leading dims)."""
        if not self.enabled:
            return
        cs = self.layers[slot]["cs"]
        if y.dtype not in UNIT_ROUNDOFF or x.shape[-1] != cs.k or y.shape[-1] != cs.n:
            return
        check_static_impl(x.reshape(-1, cs.k), y.reshape(-1, cs.n), *self.op_args(slot, with_bias))

    def _make_forward(self, mod: torch.nn.Linear):
        guard, slot = self, mod._sdcguard_slot - 1
        cs = self.layers[slot]["cs"]
        op = _op()

        def forward(x):
            b = mod.bias
            fused = b is None or x.dim() <= 2 or (x.is_contiguous() and b.dim() == 1 and b.is_contiguous())
            y = torch.nn.functional.linear(x, mod.weight, b if fused else None)
            if guard.enabled and x.numel() > 0 and y.dtype == cs.dtype:
                args = guard.op_args(slot, fused and b is not None)
                call = op if torch.compiler.is_compiling() else check_static_impl
                call(x.reshape(-1, cs.k), y.reshape(-1, cs.n), *args)
            return y if fused else y + b

        return forward

    def read_slot(self, slot: int):
        st = self._state[self.layers[slot]["device"]]
        return decode_state(st[slot:slot + 1].detach().to("cpu"))[0]

    # ---------------------------------------------------------------- results
    def poll(self, wait: bool = False) -> list:
        """Alerts since the last poll.  Without wait it never stalls: it starts a copy of the state and reports
        the previous copy once it has arrived (serve.py:1090-1129)."""
        self.stats["polls"] += 1
        events = []
        for dev, st in self._state.items():
            n = len(self.layers)
            if wait:
                pending = self._host.pop(dev, None)
                if pending is not None:
                    pending[1].synchronize()
                    events += self._report(dev, pending[0])
                host = st[:n].detach().to("cpu", copy=True)
                st[:n].zero_()
                self._next_epoch(dev, n)
                events += self._report(dev, host)
                continue
            pending = self._host.get(dev)
            if pending is not None and pending[1].query():
                events += self._report(dev, pending[0])
                self._host.pop(dev, None)
                pending = None
            if pending is None:
                buf = torch.empty((n, STATE_COLS), dtype=st.dtype, pin_memory=True)
                buf.copy_(st[:n], non_blocking=True)
                st[:n].zero_()
                self._next_epoch(dev, n)
                ev = torch.cuda.Event()
                ev.record(torch.cuda.current_stream(dev))
                self._host[dev] = (buf, ev)
        return events

    def _next_epoch(self, dev, n: int) -> None:
        cap = self._cap.get(dev)
        if cap is not None:
            cap[0][1:2].add_(1 << EPOCH_SHIFT)
            cap[0][CAP_FLAGS:CAP_FLAGS + n].zero_()
        self._epoch[dev] = self._epoch.get(dev, 0) + 1

    def mark_step(self, step: int, rows: Optional[int] = None) -> None:
        step = int(step) & STEP_MASK
        for dev in set(self._state) | set(self._cap):
            cap = self._cap.get(dev)
            if cap is not None:
                cap[0][1:2].fill_((self._epoch.get(dev, 0) << EPOCH_SHIFT) | step)

    def _report(self, dev, host: torch.Tensor) -> list:
        events = []
        rows = decode_state(host)
        counts = decode_counts(host)
        slots = [i for i, lay in enumerate(self.layers) if lay["device"] == dev and i < host.shape[0]]
        for slot in slots:
            name = self.layers[slot]["name"]
            z, flat, nz = rows[slot]
            checks, unj = counts[slot]
            self.checks_seen[name] = self.checks_seen.get(name, 0) + checks
            self.unjudged_seen[name] = self.unjudged_seen.get(name, 0) + unj
            self.stats["checks_executed"] += checks
            self.stats["unjudged_checksums"] += unj
            self.worst_seen[name] = max(self.worst_seen.get(name, 0.0), z)
            if z > self.z:
                cs = self.layers[slot]["cs"]
                bi = flat // 2
                ev = SDCEvent(detector="serve_checksum", layer=name, z=z, row=bi // cs.nb, col_block=bi % cs.nb,
                              noise=nz, nonfinite=not math.isfinite(z) or nz != nz,
                              extra={"checksum": "signed" if flat % 2 else "plain"})
                events.append(ev)
                self.events.append(ev)
                self.stats["alerts"] += 1
                if self.on_alert is not None:
                    self.on_alert(ev)
        return events

    def captured(self, dev) -> list:
        """(record, y block, x row) of every row the capture buffer kept on a device (waits for the GPU)."""
        cm, cd = self._cap[torch.device(dev)]
        head = cm[:CAP_FLAGS].cpu()
        n = min(int(head[0]), CAPTURE_SLOTS)
        recs = head[CAP_HEAD:CAP_FLAGS].view(CAPTURE_SLOTS + 1, CAP_REC)[:n].tolist()
        data = cd[:n].cpu()
        out = []
        for i, r in enumerate(recs):
            slot = r[0] // 2 - 1
            cs = self.layers[slot]["cs"]
            width = cs.bs if r[2] < cs.nbf else cs.rem
            out.append((r, data[i, :width], data[i, self._cap_w:self._cap_w + cs.k]))
        return out

    def detach(self) -> None:
        try:
            if self.layers:
                self.poll(wait=True)
        finally:
            for lay in self.layers:
                mod = lay["module"]
                if lay.get("took_over"):
                    mod.__dict__.pop("forward", None)
                mod.__dict__.pop("_sdcguard_slot", None)
                mod.__dict__.pop("_sdcguard_name", None)
            self.layers.clear()
            self._state.clear()
            self._host.clear()
            self._cap.clear()
            self.stats["layers"] = 0

