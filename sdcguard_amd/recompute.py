"""Bit fingerprints of tensors for the recompute check (reference: recompute.py:59-116, _fingerprint.py).

fingerprint(t) -> int64[3] on t's device: the sums of t's 16-bit words (8-bit for 1-byte dtypes), and of the words
times two pseudo-random odd 64-bit weights of their position (splitmix64's mix of position + 0x9E3779B97F4A7C15),
mod 2^64.  One HIP kernel pass (sdc_fingerprint3), bit-exact: wrapping integer sums do not depend on order.
"""
from __future__ import annotations

import torch

from . import _lib

# recompute.py:59-61, as signed int64 (0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9, 0x94D049BB133111EB)
_FP_SEED = -7046029254386353131
_FP_M1 = -4658895280553007687
_FP_M2 = -7723592293110705685


def fingerprint_bits(bits: torch.Tensor, start: int = 0, out: torch.Tensor = None) -> torch.Tensor:
    """The three sums of a flat int16 or int8 tensor (recompute.py:72-90's fast path, _fingerprint.py:128-130).
    With `out` ([3] int64 on the device) the sums are added into it."""
    if bits.dtype not in (torch.int16, torch.int8) or bits.dim() != 1 or not bits.is_contiguous():
        raise ValueError("fingerprint_bits takes a flat contiguous int16 or int8 tensor")
    _lib.require_gpu(bits)
    if out is None:
        out = torch.zeros(3, dtype=torch.int64, device=bits.device)
    rc = _lib.lib().sdc_fingerprint3(bits.data_ptr(), bits.numel(), bits.element_size(), int(start), out.data_ptr(),
                                     _lib.stream_of(bits))
    _lib.check(rc, "sdc_fingerprint3")
    return out


def fingerprint(t: torch.Tensor) -> torch.Tensor:
    """recompute.py:72-90: [3] int64 on t's device, no host sync."""
    x = t.detach()
    if x.numel() == 0:
        return torch.zeros(3, dtype=torch.int64, device=x.device)
    x = x.contiguous().view(-1)
    bits = x.view(torch.int16) if x.element_size() % 2 == 0 else x.view(torch.int8)
    return fingerprint_bits(bits)
