"""Column-block ABFT check of C = beta*bias + alpha*(A @ B), training flavour (oracle: test infrastructure only).

Restates checksum.py:435-530 (`_zscores`), :349-383 (`_complete_score`, `_judge_nonfinite`) and :695-725
(`resolve`) in numpy.  fp32 arithmetic follows the reference's order of operations; the expected side
``A @ B2`` is computed in float64 from the fp32 block sums and rounded once to fp32 (the reference runs an
fp32 GEMM there, cuBLAS or MKL, whose rounding is implementation-defined: the two agree to fp32 rounding).

Unlike the reference, which keeps only the worst checksum, ``zscores`` returns every checksum's score so
tests can compare the device kernel block by block.  Ties between equal worst scores resolve to the first
checksum in row-major order (torch.max on the CPU).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np

from .lowp import ABS_FLOOR, BIG, DTYPE_MAX, HALF_TINY_STEP, UNIT_ROUNDOFF
from .signs import signs as _signs

UNJUDGED = -1.0                                                    # checksum.py:346
f32 = np.float32


def l1_floor_coef(k: int) -> float:
    """checksum.py:95-104."""
    return max(1e-5, k * 2.0 ** -27)


def _f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def _sum32(x, axis) -> np.ndarray:
    return np.sum(_f32(x), axis=axis, dtype=np.float32)


def _norm2(x, axis) -> np.ndarray:
    x = _f32(x)
    with np.errstate(over="ignore", invalid="ignore"):
        return np.sqrt(np.sum(x * x, axis=axis, dtype=np.float32)).astype(np.float32)


def _norm1(x, axis) -> np.ndarray:
    return np.sum(np.abs(_f32(x)), axis=axis, dtype=np.float32)


def _amax_nan(x, axis) -> np.ndarray:
    """max |x| where NaN counts as larger than anything (torch's amax propagates NaN)."""
    a = np.abs(_f32(x))
    return np.max(a, axis=axis)            # numpy's max propagates NaN, like torch.amax


def _pair_sums(xb, s) -> np.ndarray:
    """(..., width) -> (..., 2): plain and signed fp32 sums; checksum.py:295-310."""
    xb = _f32(xb)
    return np.stack([_sum32(xb, -1), _sum32(xb * s, -1)], axis=-1)


@dataclass
class Span:
    start: int
    width: int
    nblk: int


def spans(n: int, block: int):
    """checksum.py:446-451: full blocks of bs = min(block, n), then one narrower block."""
    bs = max(1, min(block, n))
    out = []
    for start, width, nblk in ((0, bs, n // bs), ((n // bs) * bs, n % bs, 1)):
        if nblk and width:
            out.append(Span(start, width, nblk))
    return out


@dataclass
class Scores:
    z: np.ndarray          # (batch, m, nb, 2) float32 scores, every block incl. the narrower last one
    den: np.ndarray        # (batch, m, nb, 2) noise (denominator) of each checksum
    expected: np.ndarray   # (batch, m, nb, 2)
    actual: np.ndarray     # (batch, m, nb, 2)
    csb: np.ndarray        # (batch, m, nb, 2) |a_row|_2 |checksum column|_2: bound of the expected side's partial sums
    max_z: float           # after _complete_score
    batch: int
    row: int
    col_block: int
    noise: float
    unknown: bool

    @property
    def ok(self) -> bool:
        return math.isfinite(self.max_z) and self.max_z <= 6.0


def _judge_nonfinite(z, expected, actual, noise, bound, dtype, cnorm, width, step, k, unj=UNJUDGED):
    """checksum.py:359-383 (serve.py:353-368 with unj=0)."""
    with np.errstate(invalid="ignore", over="ignore"):
        e_bad = ~np.isfinite(expected)
        a_bad = ~np.isfinite(actual) & ~e_bad
        big = ~np.isfinite(noise) & ~e_bad & ~a_bad
        lim = (bound * f32(1.01)).astype(np.float32)
        z = np.where(z == z, z, f32(unj))
        z = np.where(e_bad, f32(unj), z)
        cap = (bound * f32(1.02 + k * 2.0 ** -22) + f32(step)).astype(np.float32)
        imposs = ~e_bad & ~a_bad & ~big & (lim < BIG) & (cnorm > cap * f32(math.sqrt(width)))
        z = np.where(imposs, f32(np.inf), z)
        z = np.where(a_bad, np.where(lim < min(DTYPE_MAX[dtype], BIG), f32(np.inf), f32(unj)), z)
        z = np.where(big, np.where(lim < BIG, f32(np.inf), f32(unj)), z)
    return z.astype(np.float32)


def zscores(A, B, C, bias=None, *, alpha: float = 1.0, beta: float = 1.0, block: int = 128,
            abs_floor: float = ABS_FLOOR, z: float = 6.0, dtype: str = "bf16", seed: int = 1,
            epoch: int = 0) -> Scores:
    """Every checksum's score of C = beta*bias + alpha*(A@B); A (m,k)|(bA,m,k), B (k,n)|(bB,k,n),
    C (m,n)|(b,m,n) as float32 arrays of `dtype` values.  checksum.py:435-530."""
    u = UNIT_ROUNDOFF[dtype]
    h = HALF_TINY_STEP[dtype]
    A3, B3, C3 = (_f32(t) if _f32(t).ndim == 3 else _f32(t)[None] for t in (A, B, C))
    nb_batch, m, n = C3.shape
    k = A3.shape[-1]
    if k == 0:                                         # checksum.py:386-392: one zero column
        A3 = np.zeros(A3.shape[:-1] + (1,), np.float32)
        B3 = np.zeros(B3.shape[:-2] + (1, n), np.float32)
        k = 1
    nbt = max(nb_batch, A3.shape[0], B3.shape[0])
    l1c = l1_floor_coef(k)
    A_norm = _norm2(A3, -1)[:, :, None, None]                       # (bA, m, 1, 1)
    A_l1 = _norm1(A3, -1)[:, :, None]                               # (bA, m, 1)
    zs_all, den_all, exp_all, act_all, csb_all, unknown = [], [], [], [], [], False
    for sp in spans(n, block):
        start, width, nblk = sp.start, sp.width, sp.nblk
        end = start + width * nblk
        s = _signs(width, seed, epoch)
        Cb = C3[..., start:end].reshape(nb_batch, m, nblk, width)
        Bblk = B3[..., start:end].reshape(B3.shape[0], k, nblk, width)
        B2 = _pair_sums(Bblk, s)                                     # (bB, k, nblk, 2)
        e64 = np.matmul(A3.astype(np.float64), B2.reshape(B3.shape[0], k, 2 * nblk).astype(np.float64))
        with np.errstate(over="ignore", invalid="ignore"):
            expected = e64.astype(np.float32).reshape(-1, m, nblk, 2)
            bound = (A_l1 * _amax_nan(Bblk, (-3, -1))[:, None, :]).astype(np.float32)   # (b, m, nblk)
            if alpha != 1.0:
                expected = (expected * f32(alpha)).astype(np.float32)
                bound = (bound * f32(abs(alpha))).astype(np.float32)
            if bias is not None and beta != 0:
                bias_ = _f32(bias)
                if bias_.ndim == 1:
                    bb = np.broadcast_to(bias_, (n,))[start:end].reshape(nblk, width)
                elif bias_.ndim <= 2:
                    bb = np.broadcast_to(bias_, (m, n))[:, start:end].reshape(m, nblk, width)
                else:
                    bb = np.broadcast_to(bias_, (nb_batch, m, n))[..., start:end].reshape(nb_batch, m, nblk, width)
                expected = (expected + _pair_sums(bb, s) * f32(beta)).astype(np.float32)
                bound = (bound + f32(abs(beta)) * _amax_nan(bb, -1)).astype(np.float32)
            actual = _pair_sums(Cb, s)                                   # (b, m, nblk, 2)
            cnorm = _norm2(Cb, -1)                                       # (b, m, nblk)
            noise = (cnorm * f32(u))[..., None]
            b2n = _norm2(B2, -3)[:, None]                                # (bB, 1, nblk, 2)
            b2max = _amax_nan(B2, -3)[:, None]
            bound4 = bound[..., None]
            f_l2 = ((A_norm * b2n) * f32(1e-5 * abs(alpha))).astype(np.float32)
            f_l1 = ((A_l1[..., None] * b2max) * f32(l1c * abs(alpha))).astype(np.float32)
            inf = f32(np.inf)
            floor = np.minimum(np.where(np.isfinite(f_l2), f_l2, inf), np.where(np.isfinite(f_l1), f_l1, inf))
            floor = np.where(np.isfinite(floor), floor, bound4 * f32(1e-5 * 128)).astype(np.float32)
            den = ((noise + floor) + f32(abs_floor + math.sqrt(width) * h)).astype(np.float32)
            diff = np.abs(expected - actual).astype(np.float32)
            zs = (diff / den).astype(np.float32)
            worst = (((_norm1(Cb, -1) * f32(1.25 * u)) + f32(1.25 * width * h))[..., None]
                     + floor[..., :1]) + f32(abs_floor)
            zs[..., :1] = np.minimum(zs[..., :1], diff[..., :1] / worst * f32(z))
            zs = _judge_nonfinite(zs, expected, actual, noise, bound4, dtype, cnorm[..., None], width, 2 * h, k)
        unknown = unknown or bool((zs < 0).any())
        zs_all.append(np.broadcast_to(zs, (nbt, m, nblk, 2)))
        den_all.append(np.broadcast_to(den, (nbt, m, nblk, 2)))
        exp_all.append(np.broadcast_to(expected, (nbt, m, nblk, 2)))
        act_all.append(np.broadcast_to(actual, (nbt, m, nblk, 2)))
        csb_all.append(np.broadcast_to((A_norm * b2n).astype(np.float32), (nbt, m, nblk, 2)))
    Z = np.concatenate(zs_all, axis=2)
    D = np.concatenate(den_all, axis=2)
    E = np.concatenate(exp_all, axis=2)
    Ac = np.concatenate(act_all, axis=2)
    # the reference takes the worst per span, then the worst span (first on ties), checksum.py:514-527
    best = None
    for i, zz in enumerate(zs_all):
        flat = zz.reshape(-1)
        j = int(np.argmax(flat))
        if best is None or flat[j] > best[0]:
            best = (float(flat[j]), i, j)
    mz, si, j = best
    nblk_i = zs_all[si].shape[2]
    b_i, rem = divmod(j // 2, m * nblk_i)
    r_i, c_i = divmod(rem, nblk_i)
    col_block = sum(z_.shape[2] for z_ in zs_all[:si]) + c_i
    noise_at = float(den_all[si].reshape(-1)[j])
    if unknown and mz <= z:                                            # checksum.py:349-356
        mz = UNJUDGED
    return Scores(z=Z, den=D, expected=E, actual=Ac, csb=np.concatenate(csb_all, axis=2), max_z=mz, batch=b_i, row=r_i, col_block=col_block,
                  noise=noise_at, unknown=unknown)


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


def check_matmul(A, B, C, bias=None, *, z: float = 6.0, **kw) -> CheckResult:
    """checksum.py:728-760 (the answer of `resolve` for one check)."""
    C_ = _f32(C)
    if C_.size == 0:
        return CheckResult(ok=True, max_z=0.0, nonfinite=False)
    s = zscores(A, B, C, bias, z=z, **kw)
    finite = math.isfinite(s.max_z)
    return CheckResult(ok=finite and s.max_z <= z, max_z=s.max_z, nonfinite=not finite,
                       batch=s.batch if C_.ndim == 3 else None, row=s.row, col_block=s.col_block, noise=s.noise)
