"""Sign patterns of the signed checksum (oracle: test infrastructure only).

checksum.py:239-270 (`_signs`): epoch 0 draws each block width on its own with
``torch.Generator().manual_seed((SIGN_SEED + width) % 2**63)`` and ``randint(0, 2, (width,)) * 2 - 1``;
a later epoch draws one pattern of ``max(128, width)`` with seed ``SIGN_SEED + n + 7919 * epoch`` and
narrower blocks take its prefix.  _group.py:262-291 (`_sign_table`) lays the patterns of widths
1..128 out as a 128 x 128 float table, row w-1 holding the width-w pattern (zeros after it).

The draw goes through torch's CPU generator, as the reference's does; it is not reimplemented.
"""
from __future__ import annotations

import numpy as np
import torch


def signs(width: int, seed: int, epoch: int = 0) -> np.ndarray:
    """+-1 pattern (float32) of one block width; checksum.py:252-261."""
    if epoch == 0:
        g = torch.Generator().manual_seed((seed + width) % (2 ** 63))
        s = torch.randint(0, 2, (width,), generator=g) * 2 - 1
    else:
        n = max(128, width)
        g = torch.Generator().manual_seed((seed + n + 7919 * epoch) % (2 ** 63))
        s = (torch.randint(0, 2, (n,), generator=g) * 2 - 1)[:width]
    return s.numpy().astype(np.float32)


def sign_table(seed: int, epoch: int = 0) -> np.ndarray:
    """(128, 128) float32: row w-1 = the width-w pattern, zero-padded; _group.py:276-283."""
    t = np.zeros((128, 128), dtype=np.float32)
    for w in range(1, 129):
        t[w - 1, :w] = signs(w, seed, epoch)
    return t
