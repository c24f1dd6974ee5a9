"""Weight fingerprints (reference: serve_weights.py:73-86, :151-216).

fingerprint(t) -> int64[2] on t's device: the sum of t's raw bit values x_i and the sum of x_i * k(i), mod 2^64,
with k(i) = fmix64(i ^ 0x2545F4914F6CDD1D) (MurmurHash3's finalizer); values are int16 for 2-byte dtypes, int32 for
4-byte (and the two halves of 8-byte) ones, uint8 for 1-byte ones.  One HIP kernel pass (sdc_fingerprint2).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

KEY_SEED = 0x2545F4914F6CDD1D
MIX1 = 0xFF51AFD7ED558CCD
MIX2 = 0xC4CEB9FE1A85EC53


def _int_view(t: torch.Tensor):
    """(flat integer view, kind) of a tensor's raw bits (serve_weights.py:151-161); kind as sdc_fingerprint2."""
    flat = t.detach().contiguous().view(-1)
    es = flat.element_size()
    if es == 2:
        return flat.view(torch.int16), 0
    if es == 4:
        return flat.view(torch.int32), 1
    if es == 8:
        return flat.view(torch.int64).view(torch.int32), 1
    return flat.view(torch.uint8), 2


def fingerprint(t: Optional[torch.Tensor], out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[2] int64 (serve_weights.py:172-185).  A missing or empty tensor gives zeros on the CPU."""
    if not isinstance(t, torch.Tensor) or t.numel() == 0:
        return torch.zeros(2, dtype=torch.int64)
    _lib.require_gpu(t)
    v, kind = _int_view(t)
    if out is None:
        out = torch.zeros(2, dtype=torch.int64, device=v.device)
    rc = _lib.lib().sdc_fingerprint2(v.data_ptr(), v.numel(), kind, out.data_ptr(), _lib.stream_of(v))
    _lib.check(rc, "sdc_fingerprint2")
    return out
