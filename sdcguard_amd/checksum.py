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
