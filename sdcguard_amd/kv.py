"""Paged-KV integrity: an integer fingerprint of every KV-cache block, and the check that the blocks a block table
references still hold what was recorded for them.

A block's fingerprint is recompute.fingerprint of the block as a tensor of its own (recompute.py:72-116: the sums
(b, b w1, b w2) mod 2^64 over its 16-bit words b -- 8-bit ones for a cache of 1-byte elements such as fp8,
recompute.py:86-87 -- positions numbered from 0 within the block), so it is bit-exact
against the reference's fingerprint of the same bytes.  It runs in libsdcguard_hip.so (sdc_kv_fingerprint), either
over every block of a cache or walking a block table (one entry per logical block; negative entries are unused).

What the ledger catches: a stale or reused block (the table points at a physical block whose contents are no longer
the ones recorded when that logical block was written) and any bit flip in a block's keys or values since.  It
does not see a write that recorded the wrong contents in the first place.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


def _blocks_view(cache: torch.Tensor) -> torch.Tensor:
    if cache.dim() < 2:
        raise ValueError("a paged cache has its blocks on dimension 0")
    if not cache[0].is_contiguous():
        raise ValueError("each block must be contiguous")
    return cache


def block_fingerprints(cache: torch.Tensor, ids: Optional[torch.Tensor] = None,
                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """(n, 3) int64 fingerprints of cache[ids[i]] (every block when ids is None), queued without waiting.  Rows whose
    id is negative or past the cache are zero."""
    from . import _lib
    cache = _blocks_view(cache)
    _lib.require_gpu(cache, ids)
    nblocks = cache.shape[0]
    es = cache.element_size()
    wb = 2 if es % 2 == 0 else 1                          # recompute.py:86-87: int16 words, int8 for 1-byte dtypes
    words = cache[0].numel() * es // wb
    if ids is not None:
        ids = ids.reshape(-1).to(torch.int64).contiguous()
    n = nblocks if ids is None else ids.numel()
    if out is None:
        out = torch.zeros(n, 3, dtype=torch.int64, device=cache.device)
    elif out.shape != (n, 3) or out.dtype != torch.int64:
        raise ValueError("out must be (n, 3) int64 zeros")
    rc = _lib.lib().sdc_kv_fingerprint(cache.data_ptr(), nblocks, cache.stride(0) * es, words, wb,
                                        None if ids is None else ids.data_ptr(), n, out.data_ptr(),
                                        _lib.stream_of(cache))
    _lib.check(rc, "sdc_kv_fingerprint")
    return out


@dataclass
class KVCheck:
    """A queued block-table check: per entry whether it differs from the ledger, and the count, on the device."""
    mismatch: torch.Tensor        # (R, W) bool
    count: torch.Tensor           # () int64

    def read(self) -> dict:
        bad = self.mismatch.nonzero().cpu().tolist()
        return {"mismatched": int(self.count.item()), "entries": [tuple(x) for x in bad]}


class KVLedger:
    """Fingerprints recorded per logical block (request row, block index) when the block was written, checked
    against what the block table points at now."""

    def __init__(self, cache: torch.Tensor, rows: int, width: int):
        self.cache = _blocks_view(cache)
        self.expected = torch.zeros(rows, width, 3, dtype=torch.int64, device=cache.device)
        self.known = torch.zeros(rows, width, dtype=torch.bool, device=cache.device)

    def record(self, block_table: torch.Tensor, mask: Optional[torch.Tensor] = None) -> None:
        """Record the current fingerprints of the blocks block_table (rows x width block ids, -1 for none) points
        at, for the entries in mask (default: every non-negative entry)."""
        bt = block_table.to(torch.int64)
        fp = block_fingerprints(self.cache, bt).view(*bt.shape, 3)
        m = (bt >= 0) if mask is None else (mask & (bt >= 0))
        self.expected = torch.where(m[..., None], fp, self.expected)
        self.known = self.known | m

    def verify(self, block_table: torch.Tensor) -> KVCheck:
        """Fingerprint the blocks the table points at now and compare with the recorded ones (no host sync)."""
        bt = block_table.to(torch.int64)
        fp = block_fingerprints(self.cache, bt).view(*bt.shape, 3)
        mism = self.known & (bt >= 0) & (fp != self.expected).any(-1)
        return KVCheck(mism, mism.sum())
