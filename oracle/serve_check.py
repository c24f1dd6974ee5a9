"""Serving check of one linear layer y = x @ W^T (+ b) (oracle: test infrastructure only).

``layer_constants`` restates serve.py:140-244 (`LayerChecksums`: the block sums B2 of W and the per-block
constants, computed once per layer); ``check_static`` restates serve.py:301-396 (`_check_static_impl`) and
the device kernels' scoring, _serve_fast.py:102-262 and :334-452 (`_check`, `_judge`, `_report`), with its
packed int64 state row: (bits of z << 32) | flat checksum index, (bits of z << 32) | bits of its noise, then
checks executed and unjudged checksums (serve.py:55-65).

Scores are fp32 in the reference's order of operations; the expected side x @ B2 is computed in float64
from fp32 B2 and rounded once to fp32 (the reference multiplies three bf16/fp16 parts of B2 in an fp32
GEMM: the two agree to fp32 rounding).  Where two checksums tie for the worst score, the state keeps the
larger key (the device kernels' integer maximum): the later flat index.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .abft import l1_floor_coef
from .lowp import ABS_FLOOR, BIG, DTYPE_MAX, HALF_TINY_STEP, UNIT_ROUNDOFF, split3
from .signs import signs as _signs

f32 = np.float32
STATE_COLS = 4                                                    # serve.py:64


def _f32(x):
    return np.asarray(x, dtype=np.float32)


@dataclass
class LayerConstants:
    """serve.py:140-244 for W (n x k) and bias b (n,) or None."""
    n: int
    k: int
    nb: int
    bs: int
    rem: int
    B2: np.ndarray        # (k, 2nb) fp32: column 2b = sum of block b's weight rows, 2b+1 = signed sum
    parts: np.ndarray     # (k, 6nb) in dtype: split3(B2 / scale)
    scale: np.ndarray     # (nb, 2) fp32 powers of two (fp16) or ones
    b2n: np.ndarray       # (nb, 2)
    b2max: np.ndarray     # (nb, 2)
    bmax: np.ndarray      # (nb,)
    bsum: np.ndarray      # (nb, 2)
    bmax_bias: np.ndarray  # (nb,)
    width: np.ndarray     # (nb,)
    wsq: np.ndarray       # (nb,)


def layer_constants(W, b=None, block: int = 128, dtype: str = "bf16", seed: int = 1) -> LayerConstants:
    W = _f32(W)
    n, k = W.shape
    bs = max(1, min(block, n))
    nbf, rem = n // bs, n % bs
    nb = nbf + (1 if rem else 0)
    cols = []
    if nbf:
        s = _signs(bs, seed)
        Wb = W[:nbf * bs].reshape(nbf, bs, k).astype(np.float64)
        plain = Wb.sum(axis=1)                                      # (nbf, k)
        signed = np.einsum("bjk,j->bk", Wb, s.astype(np.float64))
        cols.append(np.stack([plain, signed], axis=-1).transpose(1, 0, 2).reshape(k, 2 * nbf))
    if rem:
        s = _signs(rem, seed)
        Wr = W[nbf * bs:].astype(np.float64)
        cols.append(np.stack([Wr.sum(0), s.astype(np.float64) @ Wr], axis=-1))
    B2 = np.concatenate(cols, axis=1).astype(np.float32)           # (k, 2nb)
    with np.errstate(over="ignore", invalid="ignore"):
        b2n = np.sqrt((B2.astype(np.float64) ** 2).sum(0)).astype(np.float32).reshape(nb, 2)
        b2max = np.max(np.abs(B2), axis=0).reshape(nb, 2)
        if dtype == "fp16":
            amax = np.max(np.abs(B2), axis=0)
            ok = np.isfinite(amax) & (amax > 0)
            scale = np.where(ok, np.exp2(np.ceil(np.log2(np.maximum(amax, 1e-30)))), 1.0).astype(np.float32)
        else:
            scale = np.ones(2 * nb, dtype=np.float32)
        parts = split3((B2 / scale).astype(np.float32), dtype)
    rows_max = np.max(np.abs(W), axis=1)
    bmax = _block_reduce_max(rows_max, nbf, bs, rem)
    if b is not None:
        bf = _f32(b).astype(np.float64)
        bp = []
        if nbf:
            s = _signs(bs, seed).astype(np.float64)
            bb = bf[:nbf * bs].reshape(nbf, bs)
            bp.append(np.stack([bb.sum(1), bb @ s], axis=-1))
        if rem:
            s = _signs(rem, seed).astype(np.float64)
            br = bf[nbf * bs:]
            bp.append(np.array([[br.sum(), br @ s]]))
        bsum = np.concatenate(bp, axis=0).astype(np.float32)
        bmax_bias = _block_reduce_max(np.abs(_f32(b)), nbf, bs, rem)
    else:
        bsum = np.zeros((nb, 2), np.float32)
        bmax_bias = np.zeros(nb, np.float32)
    width = np.full(nb, float(bs), np.float32)
    if rem:
        width[-1] = float(rem)
    return LayerConstants(n=n, k=k, nb=nb, bs=bs, rem=rem, B2=B2, parts=parts, scale=scale.reshape(nb, 2),
                          b2n=b2n, b2max=b2max, bmax=bmax, bsum=bsum, bmax_bias=bmax_bias, width=width,
                          wsq=np.sqrt(width).astype(np.float32))


def _block_reduce_max(v, nbf, bs, rem):
    out = []
    if nbf:
        out.append(np.max(v[:nbf * bs].reshape(nbf, bs), axis=1))
    if rem:
        out.append(np.array([np.max(v[nbf * bs:])], np.float32))
    return np.concatenate(out).astype(np.float32)


@dataclass
class ServeScores:
    z: np.ndarray          # (m, nb, 2) scores after the Inf/NaN rules (unjudged -> 0)
    den: np.ndarray        # (m, nb, 2)
    zc: np.ndarray         # (m, nb) worse checksum's score
    sec: np.ndarray        # (m, nb) bool: the signed checksum is the worse one
    unjudged: int
    state: np.ndarray      # (4,) int64: the state row this call leaves (starting from zeros)
    expected: np.ndarray   # (m, nb, 2)
    actual: np.ndarray     # (m, nb, 2)
    csb: np.ndarray        # (m, nb, 2) |x_row|_2 |checksum column|_2: bound of the expected side's partial sums


def _bits32(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)


def check_static(x, y, c: LayerConstants, *, z: float = 6.0, abs_floor: float = ABS_FLOOR,
                 dtype: str = "bf16", seed: int = 1, with_bias: bool = True, E=None) -> ServeScores:
    """serve.py:301-396 for x (m, k), y (m, n).  E: the expected side x @ B2 (m, 2nb) before the bias sums,
    if the caller has it; else computed here in float64 and rounded to fp32."""
    x, y = _f32(x), _f32(y)
    u = UNIT_ROUNDOFF[dtype]
    h = HALF_TINY_STEP[dtype]
    m, n = y.shape
    nb, bs, k = c.nb, c.bs, x.shape[1]
    nbf, rem = n // bs, n - (n // bs) * bs
    bsum = c.bsum if with_bias else np.zeros_like(c.bsum)
    bmb = c.bmax_bias if with_bias else np.zeros_like(c.bmax_bias)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        if E is None:
            E = (x.astype(np.float64) @ c.B2.astype(np.float64)).astype(np.float32)
        expected = (_f32(E).reshape(m, nb, 2) + bsum).astype(np.float32)
        actual = np.zeros((m, nb, 2), np.float32)
        sq = np.zeros((m, nb), np.float32)
        l1 = np.zeros((m, nb), np.float32)
        for start, width, nblk in ((0, bs, nbf), (nbf * bs, rem, 1)):
            if not (nblk and width):
                continue
            s = _signs(width, seed)
            yb = y[:, start:start + width * nblk].reshape(m, nblk, width)
            j0 = start // bs
            actual[:, j0:j0 + nblk, 0] = np.sum(yb, -1, dtype=np.float32)
            actual[:, j0:j0 + nblk, 1] = np.sum(yb * s, -1, dtype=np.float32)
            sq[:, j0:j0 + nblk] = np.sum(yb * yb, -1, dtype=np.float32)
            l1[:, j0:j0 + nblk] = np.sum(np.abs(yb), -1, dtype=np.float32)
        xn = np.sqrt(np.sum(x * x, axis=1, dtype=np.float32)).reshape(m, 1, 1)
        xl1 = np.sum(np.abs(x), axis=1, dtype=np.float32).reshape(m, 1)
        bound = (xl1 * c.bmax + bmb)[..., None].astype(np.float32)             # (m, nb, 1)
        noise = (np.sqrt(sq) * f32(u))[..., None].astype(np.float32)
        f_l2 = (xn * c.b2n * f32(1e-5)).astype(np.float32)
        f_l1 = (xl1[..., None] * c.b2max * f32(l1_floor_coef(k))).astype(np.float32)
        inf = f32(np.inf)
        floor = np.minimum(np.where(np.isfinite(f_l2), f_l2, inf), np.where(np.isfinite(f_l1), f_l1, inf))
        floor = np.where(np.isfinite(floor), floor, bound * f32(1e-5 * 128)).astype(np.float32)
        den = ((noise + floor) + (f32(abs_floor) + c.wsq.reshape(1, nb, 1) * f32(h))).astype(np.float32)
        diff = np.abs(expected - actual).astype(np.float32)
        zs = (diff / den).astype(np.float32)
        worst = ((l1 * f32(1.25 * u) + f32(1.25 * h) * c.width)[..., None] + floor[..., :1]) + f32(abs_floor)
        zs = np.concatenate([np.minimum(zs[..., :1], diff[..., :1] / worst * f32(z)), zs[..., 1:]], axis=-1)
        e_bad = ~np.isfinite(expected)
        a_bad = ~np.isfinite(actual) & ~e_bad
        big = ~np.isfinite(noise) & ~e_bad & ~a_bad
        lim = (bound * f32(1.01)).astype(np.float32)
        nan = zs != zs
        zs = np.where(zs == zs, zs, f32(0))
        zs = np.where(e_bad, f32(0), zs)
        cap = (bound * f32(1.02 + k * 2.0 ** -22) + f32(2 * h)).astype(np.float32)
        imposs = ~e_bad & ~a_bad & ~big & (lim < BIG) & (noise / f32(u) > cap * c.wsq.reshape(1, nb, 1))
        zs = np.where(imposs, f32(np.inf), zs)
        lim_a = min(DTYPE_MAX[dtype], BIG)
        zs = np.where(a_bad, np.where(lim < lim_a, f32(np.inf), f32(0)), zs)
        zs = np.where(big, np.where(lim < BIG, f32(np.inf), f32(0)), zs).astype(np.float32)
        unj_mask = (nan & ~imposs & ~a_bad & ~big) | e_bad | (a_bad & ~(lim < lim_a)) | (big & ~(lim < BIG))
        unjudged = int(unj_mask.sum())
        dnan = np.where(a_bad, f32(np.nan), np.broadcast_to(den, zs.shape)).astype(np.float32)
    # the device kernels' reduction: worse checksum of each pair (plain on ties), then the largest key
    sec = zs[..., 1] > zs[..., 0]
    zc = np.where(sec, zs[..., 1], zs[..., 0]).astype(np.float32)
    dc = np.where(sec, dnan[..., 1], dnan[..., 0]).astype(np.float32)
    state = np.zeros(STATE_COLS, np.int64)
    if m > 0:
        zb = _bits32(np.maximum(zc, f32(0)))
        flat = (np.arange(m)[:, None] * nb + np.arange(nb)[None, :]) * 2 + sec.astype(np.int64)
        key_i = (zb << 32) | (flat & 0xFFFFFFFF)
        key_d = (zb << 32) | (_bits32(dc) & 0xFFFFFFFF)
        state[0] = key_i.max()
        state[1] = key_d.max()
        state[2] = 1
        state[3] = unjudged
    return ServeScores(z=zs, den=np.broadcast_to(den, zs.shape).copy(), zc=zc, sec=sec, unjudged=unjudged,
                       state=state, expected=expected, actual=actual,
                       csb=np.broadcast_to(xn * c.b2n, zs.shape).astype(np.float32))


def decode(key_i: int, key_d: int):
    """(z, flat index, noise) of a state row; _serve_fast.py:673-679."""
    zb = (int(key_i) >> 32) & 0xFFFFFFFF
    zz = np.array([zb], np.uint32).view(np.float32)[0]
    nz = np.array([int(key_d) & 0xFFFFFFFF], np.uint32).view(np.float32)[0]
    return float(zz), int(key_i) & 0xFFFFFFFF, float(nz)
