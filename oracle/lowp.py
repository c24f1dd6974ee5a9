"""bf16 / fp16 rounding of float32 arrays, in numpy (oracle: test infrastructure only).

Round to nearest, ties to even, as torch's ``Tensor.to(torch.bfloat16)`` / ``.half()`` do; NaN stays
NaN, overflow goes to +-Inf.  Values are returned as float32 arrays holding the rounded values
(every bf16 and fp16 value is exact in float32).
"""
from __future__ import annotations

import numpy as np

UNIT_ROUNDOFF = {"bf16": 2.0 ** -8, "fp16": 2.0 ** -11}          # checksum.py:75
HALF_TINY_STEP = {"bf16": 0.0, "fp16": 2.0 ** -25}                # checksum.py:83
DTYPE_MAX = {"bf16": float(np.float32(3.3895313892515355e38)), "fp16": 65504.0,
             "fp32": float(np.finfo(np.float32).max)}            # checksum.py:87-88
BIG = 1e18                                                        # checksum.py:89
ABS_FLOOR = 1e-20                                                 # checksum.py:78


def bf16_round(x) -> np.ndarray:
    """float32 -> nearest bf16 value (as float32)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    b = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(nan, np.uint32(0x7FC00000), r)
    return r.view(np.float32).reshape(a.shape)


def fp16_round(x) -> np.ndarray:
    """float32 -> nearest fp16 value (as float32); numpy's float16 cast rounds to nearest even."""
    a = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return a.astype(np.float16).astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    return bf16_round(x) if dtype == "bf16" else fp16_round(x)


def bf16_bits(x) -> np.ndarray:
    """Raw 16-bit words (uint16) of bf16 values held in float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    b = np.asarray(bits).astype(np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def split3(x, dtype: str) -> np.ndarray:
    """fp32 -> hi, mid, lo parts in `dtype`, concatenated on the last axis as the reference does, whose
    sum is x to ~2^-27 relative; checksum.py:160-166."""
    x = np.asarray(x, dtype=np.float32)
    hi = round_to(x, dtype)
    r = (x - hi).astype(np.float32)
    mid = round_to(r, dtype)
    lo = round_to((r - mid).astype(np.float32), dtype)
    return np.concatenate([hi, mid, lo], axis=-1)
