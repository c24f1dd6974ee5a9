"""Checks of quantized GEMMs (oracle: test infrastructure only).

int8 W8A8 -- modes.py:231-291 (`judge`, the int8 branch): C = A @ B with int8 A (m, k), B (k, n) and the exact
    int32 result C.  For every row and block of 128 columns the plain sum and one sum per +-1 pattern (default: the
    process's width-128 pattern, checksum._signs) must equal A @ (the same sums of B's columns) *exactly*.  The
    reference adds them in float64, exact below 2^53; here in int64.  A narrower last block (n not a multiple of
    128; modes.judge requires n % 128 == 0) uses the pattern of its own width, as every other check of the
    reference does (checksum._signs(width), seeded SIGN_SEED + width).

fp8 e4m3 with scales -- no reference function: the reference checks fp8 GEMMs only with per-tensor scale 1
    (modes.judge, fp8 branch).  Built from its pieces: for C[i, j] = sa_i * sb_j * sum_k Aq[i, k] Bq[k, j] (fp32,
    or bf16 after scaling) the column-block identity reads
        sum_{j in blk} w_j C[i, j] = sa_i * sum_k Aq[i, k] * (sum_{j in blk} w_j sb_j Bq[k, j]),
    and the noise is modes.judge's fp32-accumulator model (modes.py:276-283) with the scaled operands
        u * (C1 * |sa_i Aq_i|_2 * |(Bq sb)_blk|_F + (C2 sqrt(k) + C3 k / nfma) * |C_blk|_2)
    (plus the bf16 output rounding 2^-8 |C_blk|_2 when C is bf16), with modes.py's constants C1 = C2 = C3 = 1 and
    its unit for an fp8 tensor-core accumulation of unknown precision, u = 2^-14, nfma = 16 (modes.acc_unit /
    n_fma for GPUs other than Blackwell).  A block is wrong when z > 6, when it holds a non-finite value, or
    when an output exceeds twice |sa_i Aq_i|_2 * |sb_j Bq_j|_2 (Cauchy-Schwarz; modes.judge's `impossible`).
    With sa = sb = 1 and C fp32 this is modes.judge("fp8", ...) itself.
"""
from __future__ import annotations

import math

import numpy as np

from .signs import signs as _signs

BLOCK = 128
FP8_UNIT = 2.0 ** -14          # modes.py:49 (UNIT["fp8"]) -- acc_unit for non-Blackwell GPUs
FP8_NFMA = 16                  # modes.py:70-82 (n_fma) for GPUs other than Hopper/Blackwell
C1 = C2 = C3 = 1.0             # modes.py:48


def patterns(seed: int, width: int = BLOCK) -> np.ndarray:
    """(2, width) weights: ones, then the process's +-1 pattern of that width (modes.py:246-249 default for width
    128; checksum._signs(width) for a narrower last block)."""
    return np.stack([np.ones(width, np.int64), _signs(width, seed).astype(np.int64)])


def _block_w(W, wid: int, seed):
    """The weights of a block of `wid` columns: W itself for a full block, the width's own pattern otherwise."""
    return W[:, :wid] if wid == W.shape[1] or seed is None else patterns(seed, wid)


def _blocks(n: int):
    nbf, rem = n // BLOCK, n % BLOCK
    return nbf + (1 if rem else 0), rem


def int8_sums(A: np.ndarray, B: np.ndarray, C: np.ndarray, W: np.ndarray, seed: int = 1):
    """(actual, expected), each (m, nb, 2) int64: block sums of int32 C and A @ (block sums of B)."""
    A = A.astype(np.int64)
    B = B.astype(np.int64)
    C = C.astype(np.int64)
    m, n = C.shape
    nb, rem = _blocks(n)
    npat = W.shape[0]
    actual = np.zeros((m, nb, npat), np.int64)
    B2 = np.zeros((B.shape[0], nb, npat), np.int64)
    for b in range(nb):
        lo = b * BLOCK
        wid = rem if (b == nb - 1 and rem) else BLOCK
        w = _block_w(W, wid, seed)
        actual[:, b, :] = C[:, lo:lo + wid] @ w.T
        B2[:, b, :] = B[:, lo:lo + wid] @ w.T
    expected = (A @ B2.reshape(B.shape[0], nb * npat)).reshape(m, nb, npat)
    return actual, expected


def int8_judge(A, B, C, W, seed: int = 1) -> dict:
    """modes.judge("int8", ...): wrong_blocks and the per-block verdict (m, nb) bool."""
    actual, expected = int8_sums(A, B, C, W, seed)
    bad = (actual != expected).any(axis=-1)
    return {"wrong_blocks": int(bad.sum()), "blocks": bad.size, "bad": bad, "actual": actual,
            "expected": expected}


def fp8_e4m3_values() -> np.ndarray:
    """Every finite e4m3fn value (OCP fp8: 4 exponent bits, bias 7, 3 mantissa bits, no infinities, 0x7F/0xFF NaN)."""
    out = np.zeros(256, np.float64)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        f = b & 0x7
        if e == 0xF and f == 0x7:
            out[b] = np.nan
        elif e == 0:
            out[b] = s * f * 2.0 ** -9
        else:
            out[b] = s * (1 + f / 8.0) * 2.0 ** (e - 7)
    return out


def fp8_judge(Aq, Bq, sa, sb, C, W, *, c_bf16: bool = False, unit: float = FP8_UNIT, nfma: int = FP8_NFMA,
              z: float = 6.0, seed: int = 1) -> dict:
    """The scaled fp8 check above: per (row, block) worst z over the checksums, after the Inf/NaN and impossible
    rules (inf).  Aq, Bq: the fp8 values as float64; sa (m,), sb (n,) float; C: the result as float64."""
    Aq = np.asarray(Aq, np.float64)
    Bq = np.asarray(Bq, np.float64)
    sa = np.asarray(sa, np.float64)
    sb = np.asarray(sb, np.float64)
    C = np.asarray(C, np.float64)
    m, k = Aq.shape
    n = C.shape[1]
    nb, rem = _blocks(n)
    As = Aq * sa[:, None]
    Bs = Bq * sb[None, :]
    a_norm = np.sqrt((As ** 2).sum(1))                                   # (m,)
    b_cols = np.sqrt((Bs ** 2).sum(0))                                   # (n,)
    zout = np.zeros((m, nb))
    for b in range(nb):
        lo = b * BLOCK
        wid = rem if (b == nb - 1 and rem) else BLOCK
        w = np.asarray(_block_w(W, wid, seed), np.float64)
        cb = C[:, lo:lo + wid]
        with np.errstate(invalid="ignore", over="ignore"):
            actual = cb @ w.T                                            # (m, 2)
            expected = As @ (Bs[:, lo:lo + wid] @ w.T)
            c_norm = np.sqrt((cb ** 2).sum(1))
            b_frob = math.sqrt(float((Bs[:, lo:lo + wid] ** 2).sum()))
            per_out = C2 * math.sqrt(k) + C3 * k / nfma
            noise = unit * (C1 * a_norm * b_frob + per_out * c_norm)
            if c_bf16:
                noise = noise + 2.0 ** -8 * c_norm
            noise = noise + 1e-300
            zz = (np.abs(expected - actual) / noise[:, None]).max(axis=1)
            impossible = (np.abs(cb) > 2 * a_norm[:, None] * b_cols[None, lo:lo + wid] + 1e-300).any(axis=1)
            bad = ~np.isfinite(actual).all(axis=1) | impossible | ~np.isfinite(noise) | np.isnan(zz)
        zout[:, b] = np.where(bad, np.inf, zz)
    return {"z": zout, "wrong_blocks": int((zout > z).sum()), "worst_z": float(zout.max()) if zout.size else 0.0}
