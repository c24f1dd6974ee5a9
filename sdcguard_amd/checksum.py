"""Block checksums for matrix multiplies: constants, sign patterns and result types (reference: checksum.py).

For C = A @ B (+ bias) every block of `block` consecutive output columns must satisfy
    sum_{j in block} C[i, j] = A[i, :] . (sum_{j in block} B[:, j])        (+ the bias' block sum)
and the same with a fixed random +-1 pattern s over the block.  The residual is scored in units of the
block's estimated rounding noise; above z (default 6) it is a fault.  The arithmetic runs in the HIP library
(libsdcguard_hip.so); this module holds what the host side shares with it.
"""
from __future__ import annotations

import math
import os
import threading
from dataclasses import dataclass
from typing import Optional

import torch

# checksum.py:75-93
UNIT_ROUNDOFF = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
ABS_FLOOR = 1e-20
HALF_TINY_STEP = {torch.bfloat16: 0.0, torch.float16: 2.0 ** -25}
DTYPE_MAX = {torch.bfloat16: float(torch.finfo(torch.bfloat16).max), torch.float16: 65504.0,
             torch.float32: float(torch.finfo(torch.float32).max)}
BIG = 1e18
UNJUDGED = -1.0


def l1_floor_coef(k: int) -> float:
    """Coefficient of the expected side's rounding floor on |a_row|_1 x max|checksum column|: 1e-5, or k x 2^-27
    once that is larger (checksum.py:95-104)."""
    return max(1e-5, k * 2.0 ** -27)


@dataclass
class CheckResult:
    """checksum.py:107-122."""
    ok: bool
    max_z: float
    nonfinite: bool
    batch: Optional[int] = None
    row: Optional[int] = None
    col_block: Optional[int] = None
    noise: Optional[float] = None

    @property
    def judged(self) -> bool:
        return not (math.isfinite(self.max_z) and self.max_z < 0)


# Sign patterns (checksum.py:181-270).  SDCGUARD_SIGN_SEED pins the process's pattern (tests, replays); without it
# each process draws its own, so outputs that happen to line up with one pattern are chance, not a property.
_SIGN_SEED = int(os.environ.get("SDCGUARD_SIGN_SEED") or int.from_bytes(os.urandom(4), "little"))
_CACHE_LOCK = threading.RLock()
_SIGNS: dict = {}
_TABLES: dict = {}


def sign_seed() -> int:
    return _SIGN_SEED


def _signs(width: int, device="cpu", epoch: int = 0) -> torch.Tensor:
    """The +-1 pattern (fp32) of one block width, as checksum._signs draws it (torch's CPU generator seeded with
    SIGN_SEED + width at epoch 0; one pattern of max(128, width) seeded SIGN_SEED + n + 7919 epoch after)."""
    key = (width, str(device), epoch)
    out = _SIGNS.get(key)
    if out is not None:
        return out
    with _CACHE_LOCK:
        out = _SIGNS.get(key)
        if out is not None:
            return out
        if epoch == 0:
            g = torch.Generator().manual_seed((_SIGN_SEED + width) % (2 ** 63))
            s = (torch.randint(0, 2, (width,), generator=g) * 2 - 1).float()
        else:
            n = max(128, width)
            g = torch.Generator().manual_seed((_SIGN_SEED + n + 7919 * epoch) % (2 ** 63))
            s = (torch.randint(0, 2, (n,), generator=g) * 2 - 1).float()[:width]
        dev = torch.device(device)
        out = _SIGNS[key] = s.pin_memory().to(dev, non_blocking=True) if dev.type == "cuda" else s.to(dev)
    return out


def sign_table(device, epoch: int = 0) -> torch.Tensor:
    """(128 * 128,) fp32 on `device`: row w-1 holds the width-w pattern (_group.py:262-291).  Built once per
    device and epoch and copied without making the host wait."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    key = (str(device), epoch)
    hit = _TABLES.get(key)
    if hit is not None:
        return hit
    with _CACHE_LOCK:
        hit = _TABLES.get(key)
        if hit is not None:
            return hit
        if epoch:
            for k in [k for k in list(_TABLES) if k[1] not in (0, epoch)]:
                _TABLES.pop(k, None)
        host = torch.zeros(128, 128, dtype=torch.float32)
        for w in range(1, 129):
            host[w - 1, :w] = _signs(w, "cpu", epoch)
        host = host.reshape(-1)
        dev = host.pin_memory().to(device, non_blocking=True) if device.type == "cuda" else host.to(device)
        _TABLES[key] = dev
    return dev


def _split3(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """fp32 -> hi, mid, lo parts in `dtype` concatenated on the last axis; their sum is x to ~2^-27 relative
    (checksum.py:160-166)."""
    hi = x.to(dtype)
    r = x - hi
    mid = r.to(dtype)
    lo = (r - mid).to(dtype)
    return torch.cat([hi, mid, lo], dim=-1)


# ---------------------------------------------------------------------------------------------------------------
# The check of one matmul, queued on the GPU (checksum.py:400-432, :695-767 in the reference)

@dataclass
class CheckStat:
    """A queued check: its result row on the device plus what decoding it needs (checksum.py:125-133)."""
    result: torch.Tensor         # [3] int64: worst key (bits of z << 32 | flat), key with its noise, unjudged count
    m: int
    nb: int
    batched: bool
    z: float


def _as3(t: torch.Tensor) -> torch.Tensor:
    return t if t.dim() == 3 else t.unsqueeze(0)


def _dims3(t: torch.Tensor):
    """(batch, batch stride, rows, cols, row stride, col stride) of a 2-D or 3-D tensor (_group.py:369-373)."""
    if t.dim() == 3:
        return t.shape[0], t.stride(0), t.shape[1], t.shape[2], t.stride(1), t.stride(2)
    return 1, 0, t.shape[0], t.shape[1], t.stride(0), t.stride(1)


def matmul_zscores(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
                   alpha: float = 1.0, beta: float = 1.0, block: int = 128, abs_floor: float = ABS_FLOOR,
                   z: float = 6.0, epoch: int = 0, out: Optional[torch.Tensor] = None,
                   scores_out: Optional[torch.Tensor] = None) -> Optional[CheckStat]:
    """Queue the check of C = beta*bias + alpha*(A @ B) on the GPU without waiting (checksum.py:400-432).  2-D
    (mm/addmm) or 3-D (bmm/baddbmm).  None when C's dtype isn't bf16/fp16.  `out`: a [3] int64 device tensor of
    zeros to receive the result (a fresh one otherwise)."""
    from . import _lib
    if C.dtype not in UNIT_ROUNDOFF:
        return None
    if C.numel() == 0:
        raise ValueError("empty output: nothing to check (callers skip these, see is_empty)")
    _lib.require_gpu(A, B, C, bias)
    dt = C.dtype
    if A.shape[-1] == 0:                                   # checksum.py:386-392: one zero column
        A = A.new_zeros(*A.shape[:-1], 1)
        B = B.new_zeros(*B.shape[:-2], 1, B.shape[-1])
    A = A if A.dtype == dt else A.to(dt)
    B = B if B.dtype == dt else B.to(dt)
    ba, sab, m, k, sam, sak = _dims3(A)
    bb, sbb, kb, n, sbk, sbn = _dims3(B)
    bc, scb, mc, nc, scm, scn = _dims3(C)
    if mc != m or kb != k or nc != n:
        raise ValueError(f"shape mismatch: A{tuple(A.shape)} B{tuple(B.shape)} C{tuple(C.shape)}")
    nbt = max(ba, bb)
    if bc != nbt and not (ba == 1 and bb == 1):
        raise ValueError(f"batch mismatch: A{tuple(A.shape)} B{tuple(B.shape)} C{tuple(C.shape)}")
    if ba == 1 and bb == 1 and bc > 1:                    # (a batched C of a 2-D product: check each batch)
        raise ValueError("a 3-D output needs 3-D operands")
    bs = max(1, min(block, n))
    if bs > 128:
        raise _lib.HipLibraryError(f"blocks up to 128 wide, not {bs}")
    kind, b_ptr, sb_b, sb_m, sb_n = 0, None, 0, 0, 0
    if bias is not None and beta != 0:
        bias = bias if bias.dtype == dt else bias.to(dt)
        if bias.dim() == 1 and bias.numel() in (1, n):
            kind, b_ptr, sb_n = 1, bias, (0 if bias.numel() == 1 else bias.stride(0))
        else:
            full = torch.broadcast_to(bias, (bc, m, n)) if bias.dim() == 3 or C.dim() == 3 else \
                torch.broadcast_to(bias, (m, n)).unsqueeze(0)
            kind, b_ptr = 2, full
            sb_b, sb_m, sb_n = full.stride(0) if C.dim() == 3 else 0, full.stride(1), full.stride(2)
    if out is None:
        out = torch.zeros(3, dtype=torch.int64, device=C.device)
    L = _lib.lib()
    ws_bytes = int(L.sdc_matmul_check_workspace(ba, bb, m, k, n, bs))
    ws = _lib.workspace(C.device, ws_bytes)
    rc = L.sdc_matmul_check(
        _lib.dtype_code(dt), A.data_ptr(), sab, sam, sak, ba, B.data_ptr(), sbb, sbk, sbn, bb,
        C.data_ptr(), scb, scm, scn, bc, m, k, n, bs, None if b_ptr is None else b_ptr.data_ptr(), kind,
        sb_b, sb_m, sb_n, float(alpha), float(beta), float(z), float(abs_floor),
        sign_table(C.device, epoch).data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes,
        None if scores_out is None else scores_out.data_ptr(), _lib.stream_of(C))
    _lib.check(rc, "sdc_matmul_check")
    nb = -(-n // bs)
    return CheckStat(result=out, m=m, nb=nb, batched=C.dim() == 3, z=float(z))


# The precise check of an fp32 output (checksum.py:537-563): u = 2^-24 and the noise model's constants.
ACC_UNIT = 2.0 ** -24
ACC_C1, ACC_C2, ACC_C3 = 0.6, 1.0, 1.0


def acc_supported(A: torch.Tensor, C: torch.Tensor) -> bool:
    """The precise check takes an fp32 C of bf16/fp16 operands (checksum.py:563-564)."""
    return C.dtype == torch.float32 and A.dtype in UNIT_ROUNDOFF


def matmul_zscores_acc(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
                       alpha: float = 1.0, beta: float = 1.0, block: int = 128, abs_floor: float = ABS_FLOOR,
                       z: float = 6.0, nfma: Optional[int] = None, epoch: int = 0,
                       out: Optional[torch.Tensor] = None,
                       scores_out: Optional[torch.Tensor] = None) -> Optional[CheckStat]:
    """Queue the precise check of C = beta*bias + alpha*(A @ B), C the fp32 result (not rounded), A and B bf16/fp16
    (checksum.py:587-607): float64 checksums against the fp32 accumulation's rounding.  Same result row and read-back
    as matmul_zscores (resolve() decodes both).  None if the dtypes don't fit.  nfma: tensor-core products per
    truncation step (None: no tensor cores)."""
    from . import _lib
    if not acc_supported(A, C):
        return None
    if C.numel() == 0:
        raise ValueError("empty output: nothing to check (callers skip these, see is_empty)")
    _lib.require_gpu(A, B, C, bias)
    dt = A.dtype
    if A.shape[-1] == 0:                                   # checksum.py:386-392: one zero column
        A = A.new_zeros(*A.shape[:-1], 1)
        B = B.new_zeros(*B.shape[:-2], 1, B.shape[-1])
    B = B if B.dtype == dt else B.to(dt)
    ba, sab, m, k, sam, sak = _dims3(A)
    bb, sbb, kb, n, sbk, sbn = _dims3(B)
    bc, scb, mc, nc, scm, scn = _dims3(C)
    if mc != m or kb != k or nc != n:
        raise ValueError(f"shape mismatch: A{tuple(A.shape)} B{tuple(B.shape)} C{tuple(C.shape)}")
    if ba not in (1, bc) or bb not in (1, bc) or (bc > 1 and ba == 1 and bb == 1):
        raise ValueError(f"batch mismatch: A{tuple(A.shape)} B{tuple(B.shape)} C{tuple(C.shape)}")
    bs = max(1, min(block, n))
    if bs > 128:
        raise _lib.HipLibraryError(f"blocks up to 128 wide, not {bs}")
    kind, b_ptr, sb_b, sb_m, sb_n = 0, None, 0, 0, 0
    if bias is not None and beta != 0:
        if bias.dtype not in (dt, torch.float32):
            bias = bias.float()
        if bias.dim() == 1 and bias.numel() in (1, n):
            kind, b_ptr, sb_n = 1, bias, (0 if bias.numel() == 1 else bias.stride(0))
        else:
            full = torch.broadcast_to(bias, (bc, m, n)) if bias.dim() == 3 or C.dim() == 3 else \
                torch.broadcast_to(bias, (m, n)).unsqueeze(0)
            kind, b_ptr = 2, full
            sb_b, sb_m, sb_n = full.stride(0) if C.dim() == 3 else 0, full.stride(1), full.stride(2)
        if b_ptr.dtype == torch.float32:
            kind |= 4
    if out is None:
        out = torch.zeros(3, dtype=torch.int64, device=C.device)
    L = _lib.lib()
    ws_bytes = int(L.sdc_matmul_check_acc_workspace(ba, bb, bc, m, k, n, bs))
    ws = _lib.workspace(C.device, ws_bytes)
    rc = L.sdc_matmul_check_acc(
        _lib.dtype_code(dt), A.data_ptr(), sab, sam, sak, ba, B.data_ptr(), sbb, sbk, sbn, bb,
        C.data_ptr(), scb, scm, scn, bc, m, k, n, bs, None if b_ptr is None else b_ptr.data_ptr(), kind,
        sb_b, sb_m, sb_n, float(alpha), float(beta), float(nfma or 0), float(z), float(abs_floor),
        sign_table(C.device, epoch).data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes,
        None if scores_out is None else scores_out.data_ptr(), _lib.stream_of(C))
    _lib.check(rc, "sdc_matmul_check_acc")
    nb = -(-n // bs)
    return CheckStat(result=out, m=m, nb=nb, batched=C.dim() == 3, z=float(z))


def check_matmul_acc(A, B, C, bias=None, *, z: float = 6.0, nfma: Optional[int] = None, **kw) -> Optional[CheckResult]:
    """matmul_zscores_acc, answered now (checksum.py:689-694).  None if the dtypes don't fit."""
    if C.numel() == 0 and acc_supported(A, C):
        return CheckResult(ok=True, max_z=0.0, nonfinite=False)
    st = matmul_zscores_acc(A, B, C, bias, z=z, nfma=nfma, **kw)
    return None if st is None else resolve([st], z)[0]


def _f32_of_bits(b: int) -> float:
    import struct
    return struct.unpack("<f", struct.pack("<I", b & 0xFFFFFFFF))[0]


def resolve(stats, z: float = 6.0) -> list:
    """Read queued checks back (one transfer per device for all of them) and decode them (checksum.py:695-725)."""
    if not stats:
        return []
    rows = [None] * len(stats)
    by_device: dict = {}
    for i, s in enumerate(stats):
        by_device.setdefault(s.result.device, []).append(i)
    for idx in by_device.values():
        host = torch.stack([stats[i].result for i in idx]).cpu().tolist()
        for j, i in enumerate(idx):
            rows[i] = host[j]
    out = []
    for s, (key, keyd, unjudged) in zip(stats, rows):
        mz = _f32_of_bits(key >> 32)
        flat = key & 0xFFFFFFFF
        noise = _f32_of_bits(keyd)
        if unjudged and mz <= z:                          # checksum.py:349-356
            mz = UNJUDGED
        blk = flat // 2
        b_i, rem = divmod(blk, s.m * s.nb)
        r_i, c_i = divmod(rem, s.nb)
        finite = math.isfinite(mz)
        out.append(CheckResult(ok=finite and mz <= z, max_z=mz, nonfinite=not finite,
                               batch=b_i if s.batched else None, row=r_i, col_block=c_i, noise=noise))
    return out


def is_empty(C: torch.Tensor) -> bool:
    return C.numel() == 0


def check_matmul(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
                 alpha: float = 1.0, beta: float = 1.0, block: int = 128, z: float = 6.0,
                 abs_floor: float = ABS_FLOOR, epoch: int = 0) -> Optional[CheckResult]:
    """Check C = beta*bias + alpha*(A @ B) and answer now (checksum.py:728-760).  None if the dtype is unsupported."""
    if is_empty(C) and C.dtype in UNIT_ROUNDOFF:
        return CheckResult(ok=True, max_z=0.0, nonfinite=False)
    st = matmul_zscores(A, B, C, bias, alpha=alpha, beta=beta, block=block, abs_floor=abs_floor, z=z, epoch=epoch)
    return None if st is None else resolve([st], z)[0]


def check_linear(x, weight, bias, y, **kw) -> Optional[CheckResult]:
    """Check y = torch.nn.functional.linear(x, weight, bias) for any leading dims (checksum.py:763-767)."""
    return check_matmul(x.reshape(-1, x.shape[-1]), weight.t(), y.reshape(-1, y.shape[-1]), bias, **kw)


def linear_rows_operands(x, weight, bias, y):
    """(A, B, C, bias) of the row-block check of y = linear(x, weight, bias): for every output column j and block of
    `block` rows, sum_{i in blk} s_i y[i, j] = (sum_{i in blk} s_i x[i, :]) . weight[j, :] + (sum s_i) bias[j].  That is
    the column-block check of y^T = weight @ x^T + bias[:, None] (the reference's own identity applied to the
    transposed product; every operand is a strided view, nothing is copied)."""
    x2 = x.reshape(-1, x.shape[-1])
    y2 = y.reshape(-1, y.shape[-1])
    b = None if bias is None else bias.reshape(-1, 1)
    return weight, x2.t(), y2.t(), b


def check_linear_rows(x, weight, bias, y, **kw) -> Optional[CheckResult]:
    """Row-block check of y = torch.nn.functional.linear(x, weight, bias).  The result's `row` is the output column
    and `col_block` the block of token rows."""
    return check_matmul(*linear_rows_operands(x, weight, bias, y), **kw)


def _bias_fits(bias: Optional[torch.Tensor], shape) -> bool:
    """A shared bias applies to a group's output when it broadcasts to exactly that shape."""
    if bias is None:
        return True
    try:
        return tuple(torch.broadcast_shapes(tuple(bias.shape), tuple(shape))) == tuple(shape)
    except RuntimeError:
        return False


# how a torch._grouped_mm layout (a.dim(), b.dim()) splits into per-group products: group g, its rows or columns
# [lo, hi) -> (A, B, C); and whether an empty group still has an output to check (grouped along k: out[g] is zeros)
_GROUP_SLICES = {
    (2, 3): (lambda a, b, out, g, lo, hi: (a[lo:hi], b[g], out[lo:hi]), False),          # tokens by expert
    (3, 2): (lambda a, b, out, g, lo, hi: (a[g], b[:, lo:hi], out[:, lo:hi]), False),    # grouped along n
    (2, 2): (lambda a, b, out, g, lo, hi: (a[:, lo:hi], b[lo:hi, :], out[g]), True),     # grouped along k
}


def grouped_checks(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, offs: Optional[torch.Tensor],
                   bias: Optional[torch.Tensor] = None) -> list:
    """The (A, B, C, bias, alpha, beta) checks of a torch._grouped_mm result, as the reference's guard splits one
    (guard.py:102-143): groups cut at the cumulative ends `offs` (read on the host), a 3-D x 3-D product as one
    batched check, and no check for a group whose output the shared bias does not broadcast to."""
    if a.dim() == 3 and b.dim() == 3:
        return [(a, b, out, bias, 1.0, 1.0)] if _bias_fits(bias, out.shape[1:]) else []
    layout = _GROUP_SLICES.get((a.dim(), b.dim()))
    if layout is None or offs is None:
        return []
    cut, keep_empty = layout
    bounds = [0] + [int(e) for e in offs.tolist()]
    found = []
    for g in range(len(bounds) - 1):
        lo, hi = bounds[g], bounds[g + 1]
        if hi <= lo and not keep_empty:
            continue
        A, B, C = cut(a, b, out, g, lo, max(lo, hi))
        if _bias_fits(bias, C.shape):
            found.append((A, B, C, bias, 1.0, 1.0))
    return found


@dataclass
class GroupedStat:
    """A queued grouped check: one result row per group on the device (worst key over the group's rows, key with its
    noise, unjudged count) and what decoding it needs."""
    results: torch.Tensor        # (groups, 3) int64
    offs: torch.Tensor           # the group ends as the kernels read them (clamped, non-decreasing; device)
    rows: int
    nb: int
    z: float


def grouped_zscores(a: torch.Tensor, b: Optional[torch.Tensor], out: torch.Tensor, offs: torch.Tensor,
                    bias: Optional[torch.Tensor] = None, *, block: int = 128, abs_floor: float = ABS_FLOOR,
                    z: float = 6.0, epoch: int = 0, scores_out: Optional[torch.Tensor] = None,
                    checksums: Optional["GroupedChecksums"] = None) -> GroupedStat:
    """Queue the check of a MoE grouped product out = a @ b[g] for the rows of group g (a: (T, k) tokens sorted by
    expert, b: (G, k, n), out: (T, n), offs: (G,) cumulative row ends, int32 or int64, on the device) without
    reading offs on the host: every group's rows are checked against that group's B, as
    check_matmul(a[start:end], b[g], out[start:end]) checks them (guard._grouped_checks + checksum._zscores).
    checksums: the layer's GroupedChecksums (b and bias may then be None; block and epoch are theirs)."""
    from . import _lib
    if checksums is not None:
        return _grouped_with(a, checksums, out, offs, abs_floor, z, scores_out)
    if a.dim() != 2 or b.dim() != 3 or out.dim() != 2:
        raise ValueError("grouped_zscores covers the (T, k) x (G, k, n) -> (T, n) layout")
    _lib.require_gpu(a, b, out, offs, bias)
    dt = out.dtype
    if dt not in UNIT_ROUNDOFF:
        raise ValueError(f"unsupported output dtype {dt}")
    T, k = a.shape
    G, kb, n = b.shape
    if kb != k or out.shape != (T, n) or offs.numel() != G:
        raise ValueError(f"shape mismatch: a{tuple(a.shape)} b{tuple(b.shape)} out{tuple(out.shape)} offs {offs.numel()}")
    a = a if a.dtype == dt else a.to(dt)
    b = b if b.dtype == dt else b.to(dt)
    if bias is not None:
        bias = bias.reshape(-1)
        if bias.numel() != n:
            raise ValueError("grouped_zscores: a shared bias of n values")
        bias = bias if bias.dtype == dt else bias.to(dt)
    # (a private copy of the ends, so a routing buffer reused before resolve_grouped does not change how the results
    # decode)
    offs64 = _clamped_ends(offs, T)
    L = _lib.lib()
    nb = -(-n // block)
    results = torch.zeros(G, 3, dtype=torch.int64, device=out.device)
    ws = _lib.workspace(out.device, int(L.sdc_grouped_check_workspace(G, T, k, n, block)))
    rc = L.sdc_grouped_check(_lib.dtype_code(dt), a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0),
                             b.stride(1), b.stride(2), G, out.data_ptr(), out.stride(0), out.stride(1), T, k, n, block,
                             offs64.data_ptr(), None if bias is None else bias.data_ptr(),
                             0 if bias is None else bias.stride(0), float(z), float(abs_floor),
                             sign_table(out.device, epoch).data_ptr(), results.data_ptr(), ws.data_ptr(), ws.numel(),
                             None if scores_out is None else scores_out.data_ptr(), _lib.stream_of(out))
    _lib.check(rc, "sdc_grouped_check")
    return GroupedStat(results, offs64, T, nb, z)


class GroupedChecksums:
    """A served MoE layer's grouped-check constants, made once on the device from its expert weights (groups, k, n)
    and optional shared bias (n,): every expert's block sums, their norms, maxima and scales, and the three 16-bit
    parts of the scaled sums (sdc_grouped_constants).  grouped_zscores(..., checksums=this) then runs only the
    expected-side GEMM and the pass over the output, with the same results as a call that makes them (this
    library's serving form; the reference makes every expert's block sums in every call).  The constants follow the
    weights they were made from: make them again after the weights change."""

    def __init__(self, b: torch.Tensor, bias: Optional[torch.Tensor] = None, *, block: int = 128, epoch: int = 0):
        from . import _lib
        if b.dim() != 3:
            raise ValueError("GroupedChecksums takes expert weights (groups, k, n)")
        _lib.require_gpu(b, bias)
        if b.dtype not in UNIT_ROUNDOFF:
            raise ValueError(f"unsupported dtype {b.dtype}")
        G, k, n = b.shape
        self.groups, self.k, self.n, self.block, self.epoch, self.dtype = G, k, n, block, epoch, b.dtype
        if bias is not None:
            bias = bias.reshape(-1)
            if bias.numel() != n:
                raise ValueError("GroupedChecksums: a shared bias of n values")
            bias = bias if bias.dtype == b.dtype else bias.to(b.dtype)
        self.has_bias = bias is not None
        L = _lib.lib()
        nbytes = int(L.sdc_grouped_constants_bytes(G, k, n, block))
        if nbytes <= 0:
            raise ValueError(f"GroupedChecksums: unsupported shape {tuple(b.shape)} or block {block}")
        self.consts = torch.empty(nbytes // 4 + 64, dtype=torch.float32, device=b.device)
        off = (-self.consts.data_ptr()) % 256 // 4          # 256-byte aligned start
        self._ptr = self.consts.data_ptr() + 4 * off
        ws = _lib.workspace(b.device, int(L.sdc_grouped_constants_workspace(G, k, n, block)))
        rc = L.sdc_grouped_constants(_lib.dtype_code(b.dtype), b.data_ptr(), b.stride(0), b.stride(1), b.stride(2),
                                     G, k, n, block, None if bias is None else bias.data_ptr(),
                                     0 if bias is None else bias.stride(0), sign_table(b.device, epoch).data_ptr(),
                                     self._ptr, nbytes, ws.data_ptr(), ws.numel(), _lib.stream_of(b))
        _lib.check(rc, "sdc_grouped_constants")


def _clamped_ends(offs: torch.Tensor, T: int) -> torch.Tensor:
    # the ends as both kernels read them: clamped to the rows and made non-decreasing (a running maximum), so the
    # GEMM's tile walk and the scoring pass's row-to-group search agree whatever offs holds; a private copy
    return torch.cummax(offs.reshape(-1).to(torch.int64).clamp(0, T), 0).values.contiguous()


def _grouped_with(a, cs: "GroupedChecksums", out, offs, abs_floor, z, scores_out) -> GroupedStat:
    from . import _lib
    if a.dim() != 2 or out.dim() != 2:
        raise ValueError("grouped_zscores covers the (T, k) x (G, k, n) -> (T, n) layout")
    _lib.require_gpu(a, out, offs, cs.consts)
    dt = out.dtype
    if dt != cs.dtype:
        raise ValueError(f"the output's dtype {dt} is not the checksums' {cs.dtype}")
    T, k = a.shape
    G, n = cs.groups, cs.n
    if k != cs.k or out.shape != (T, n) or offs.numel() != G:
        raise ValueError(f"shape mismatch: a{tuple(a.shape)} out{tuple(out.shape)} offs {offs.numel()} for "
                         f"checksums of ({G}, {cs.k}, {n})")
    a = a if a.dtype == dt else a.to(dt)
    offs64 = _clamped_ends(offs, T)
    L = _lib.lib()
    results = torch.zeros(G, 3, dtype=torch.int64, device=out.device)
    ws = _lib.workspace(out.device, int(L.sdc_grouped_check_consts_workspace(G, T, k, n, cs.block)))
    rc = L.sdc_grouped_check_consts(_lib.dtype_code(dt), a.data_ptr(), a.stride(0), a.stride(1), cs._ptr, G,
                                    out.data_ptr(), out.stride(0), out.stride(1), T, k, n, cs.block, offs64.data_ptr(),
                                    1 if cs.has_bias else 0, float(z), float(abs_floor),
                                    sign_table(out.device, cs.epoch).data_ptr(), results.data_ptr(), ws.data_ptr(),
                                    ws.numel(), None if scores_out is None else scores_out.data_ptr(),
                                    _lib.stream_of(out))
    _lib.check(rc, "sdc_grouped_check_consts")
    return GroupedStat(results, offs64, T, -(-n // cs.block), z)


def resolve_grouped(st: GroupedStat) -> list:
    """One CheckResult per non-empty group, in group order (the checks guard._grouped_checks makes), rows relative to
    the group's first row as check_matmul on the group's slice reports them (two small device-to-host copies)."""
    ends = [int(e) for e in st.offs.tolist()]
    host = st.results.cpu().tolist()
    out, start = [], 0
    for g, end in enumerate(ends):
        end = min(end, st.rows)
        if end > start:
            key, keyd, unjudged = host[g]
            mz = _f32_of_bits(key >> 32)
            if unjudged and mz <= st.z:
                mz = UNJUDGED
            flat = key & 0xFFFFFFFF
            r_i, c_i = divmod(flat // 2, st.nb)
            finite = math.isfinite(mz)
            out.append(CheckResult(ok=finite and mz <= st.z, max_z=mz, nonfinite=not finite, batch=None,
                                   row=(r_i - start) if key else 0, col_block=c_i, noise=_f32_of_bits(keyd)))
        start = max(start, end)
    return out


def check_grouped_mm(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, offs: Optional[torch.Tensor] = None,
                     bias: Optional[torch.Tensor] = None, **kw) -> list:
    """Check a torch._grouped_mm result: one CheckResult per check guard._grouped_checks would make.  The MoE
    forward layout (2-D x 3-D) runs as one device-side grouped check; the others as one check per group."""
    device_path = {"block", "abs_floor", "z", "epoch", "scores_out"}
    if a.dim() == 2 and b.dim() == 3 and offs is not None and out.dtype in UNIT_ROUNDOFF and \
            (bias is None or bias.numel() == out.shape[-1]) and set(kw) <= device_path:
        return resolve_grouped(grouped_zscores(a, b, out, offs, bias, **kw))
    res = []
    for A, B, C, bi, al, be in grouped_checks(a, b, out, offs, bias):
        res.append(check_matmul(A, B, C, bi, alpha=al, beta=be, **kw))
    return res
