"""The column-block check's scores in torch on the CPU (oracle: test infrastructure only).

The CPU baseline that the benchmark times next to the GPU check: the reference's own torch path, checksum.py:435-530
(`_zscores`) with :359-383 (`_judge_nonfinite`), run on CPU tensors on every host core.  The arithmetic is
oracle.abft.zscores' (which pins it: tests/test_oracle_torch.py compares the two on random and faulted problems),
except that the expected side is an fp32 GEMM (torch.matmul: oneDNN/MKL on the CPU), as the reference computes it.
Only what the benchmark's workloads need is restated: 2-D operands, alpha = beta = 1, a 1-D bias or none.

The row-block check of a linear layer y = x W^T + b is this column-block check of y^T = W x^T + b[:, None]; the
benchmark runs it as `zscores(W, x.T, y.T, b[:, None])`.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .abft import l1_floor_coef, spans
from .lowp import ABS_FLOOR, BIG, DTYPE_MAX, HALF_TINY_STEP, UNIT_ROUNDOFF
from .signs import signs as _signs

UNJUDGED = -1.0


def _pair_sums(xb: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """(..., width) -> (..., 2): plain and signed fp32 sums; checksum.py:295-310."""
    return torch.stack([xb.sum(-1), (xb * s).sum(-1)], dim=-1)


def _judge_nonfinite(z, expected, actual, noise, bound, dtype, cnorm, width, step, k):
    """checksum.py:359-383."""
    e_bad = ~torch.isfinite(expected)
    a_bad = ~torch.isfinite(actual) & ~e_bad
    big = ~torch.isfinite(noise) & ~e_bad & ~a_bad
    lim = bound * 1.01
    z = torch.where(z == z, z, torch.full_like(z, UNJUDGED))
    z = torch.where(e_bad, torch.full_like(z, UNJUDGED), z)
    cap = bound * (1.02 + k * 2.0 ** -22) + step
    imposs = ~e_bad & ~a_bad & ~big & (lim < BIG) & (cnorm > cap * math.sqrt(width))
    inf = torch.full_like(z, math.inf)
    z = torch.where(imposs, inf, z)
    z = torch.where(a_bad, torch.where(lim < min(DTYPE_MAX[dtype], BIG), inf, torch.full_like(z, UNJUDGED)), z)
    return torch.where(big, torch.where(lim < BIG, inf, torch.full_like(z, UNJUDGED)), z)


def zscores(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
            block: int = 128, abs_floor: float = ABS_FLOOR, z: float = 6.0, dtype: str = "bf16", seed: int = 1,
            epoch: int = 0):
    """Scores of every checksum of C = A @ B (+ bias), A (m, k), B (k, n), C (m, n) CPU tensors of `dtype` values
    (any float dtype; computed in fp32).  bias: (n,) or (m, 1).  Returns (z (m, nb, 2), worst z, (row, block))."""
    u, h = UNIT_ROUNDOFF[dtype], HALF_TINY_STEP[dtype]
    A, B, C = A.float(), B.float(), C.float()
    m, k = A.shape
    n = C.shape[1]
    l1c = l1_floor_coef(k)
    A_norm = A.pow(2).sum(-1).sqrt()[:, None, None]                    # (m, 1, 1)
    A_l1 = A.abs().sum(-1)[:, None]                                     # (m, 1)
    out = []
    for sp in spans(n, block):
        start, width, nblk = sp.start, sp.width, sp.nblk
        end = start + width * nblk
        s = torch.from_numpy(_signs(width, seed, epoch))
        Cb = C[:, start:end].reshape(m, nblk, width)
        Bblk = B[:, start:end].reshape(k, nblk, width)
        B2 = _pair_sums(Bblk, s)                                        # (k, nblk, 2)
        expected = (A @ B2.reshape(k, 2 * nblk)).reshape(m, nblk, 2)
        bound = A_l1 * Bblk.abs().amax(dim=(0, 2))[None, :]             # (m, nblk)
        if bias is not None:
            bb = bias.float()
            bb = bb[start:end].reshape(nblk, width) if bb.dim() == 1 else \
                bb.expand(m, n)[:, start:end].reshape(m, nblk, width)
            expected = expected + _pair_sums(bb, s)
            bound = bound + bb.abs().amax(-1)
        actual = _pair_sums(Cb, s)
        cnorm = Cb.pow(2).sum(-1).sqrt()                                 # (m, nblk)
        noise = (cnorm * u)[..., None]
        b2n = B2.pow(2).sum(0).sqrt()[None]                              # (1, nblk, 2)
        b2max = B2.abs().amax(0)[None]
        bound4 = bound[..., None]
        f_l2 = (A_norm * b2n) * 1e-5
        f_l1 = (A_l1[..., None] * b2max) * l1c
        inf = torch.full_like(f_l2, math.inf)
        floor = torch.minimum(torch.where(torch.isfinite(f_l2), f_l2, inf), torch.where(torch.isfinite(f_l1), f_l1, inf))
        floor = torch.where(torch.isfinite(floor), floor, bound4 * (1e-5 * 128))
        den = (noise + floor) + (abs_floor + math.sqrt(width) * h)
        diff = (expected - actual).abs()
        zs = diff / den
        worst = ((Cb.abs().sum(-1) * (1.25 * u)) + 1.25 * width * h)[..., None] + floor[..., :1] + abs_floor
        zs = torch.cat([torch.minimum(zs[..., :1], diff[..., :1] / worst * z), zs[..., 1:]], dim=-1)
        zs = _judge_nonfinite(zs, expected, actual, noise, bound4, dtype, cnorm[..., None], width, 2 * h, k)
        out.append(zs)
    Z = torch.cat(out, dim=1)
    j = int(torch.argmax(Z.reshape(-1)))
    worst_z = float(Z.reshape(-1)[j])
    if bool((Z < 0).any()) and worst_z <= z:
        worst_z = UNJUDGED
    nb = Z.shape[1]
    return Z, worst_z, ((j // 2) // nb, (j // 2) % nb)


def linear_both(x: torch.Tensor, W: torch.Tensor, b: Optional[torch.Tensor], y: torch.Tensor, **kw):
    """Both block checks of y = x W^T + b: (column-block result, row-block result), each as zscores returns."""
    col = zscores(x, W.t(), y, b, **kw)
    row = zscores(W, x.t(), y.t(), None if b is None else b[:, None], **kw)
    return col, row
