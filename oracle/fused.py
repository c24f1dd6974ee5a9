"""The precise check fused into the matmul (oracle: test infrastructure only; never imported by the library).

Restates fused.py in numpy:
  * block_stats       fused.py:108-114 (the statistics epilogue of `_fused_linear_kernel`): per row and block of 128
                      columns of the fp32 accumulator (bias added), the float64 plain sum, signed sum, sum of squares
                      and sum of absolute values;
  * zscores_from_stats  fused.py:181-235: precise mode's check (checksum._acc_zscores) with C's block sums taken
                      from those statistics;
  * block_sum_parts   fused.py:262-316 (`_pow2_scale`, `_bside_kernel`): each block sum of B split in three 16-bit
                      parts (fp16: divided first by a power of two), and the block's W-side norms;
  * checked_scores    fused.py:392-458 (the epilogue of `_fused_check_kernel`): the fp32 self-check's score of every
                      block, from the actual side's statistics and the expected side.
The reference sums in fp32 where this restatement (and the HIP kernels) sum in float64 and round once: block sums of
B, the accumulator's block sums and the expected side differ from the reference's by its own rounding, which its
noise model covers (tests bound that difference by the model's terms).
"""
from __future__ import annotations

import math

import numpy as np

from .abft import _amax_nan, _f32, _judge_nonfinite, _norm2, spans
from .acc import ACC_C1, ACC_C2, ACC_C3, ACC_UNIT, Scores, _pair_sums64
from .lowp import ABS_FLOOR
from .signs import signs as _signs

BLOCK = 128
BIG = 1e18
F32_MAX = float(np.finfo(np.float32).max)
f32 = np.float32


def signs_for(n: int, seed: int = 1, epoch: int = 0) -> np.ndarray:
    """The +-1 pattern of every output column: full blocks' pattern repeated, then the narrower last block's own
    (fused.py:49-65)."""
    nfull, rem = divmod(n, BLOCK)
    parts = [np.tile(_signs(BLOCK, seed, epoch), nfull)] if nfull else []
    if rem:
        parts.append(_signs(rem, seed, epoch))
    return np.concatenate(parts).astype(np.float64) if parts else np.zeros(0)


def block_stats(C, *, seed: int = 1, epoch: int = 0) -> np.ndarray:
    """(m, n) accumulator (fp32 or float64 values) -> (m, ceil(n/128), 4) float64 (fused.py:108-114)."""
    C = np.asarray(C, np.float64)
    m, n = C.shape
    nb = -(-n // BLOCK)
    pad = np.zeros((m, nb * BLOCK))
    pad[:, :n] = C
    s = np.zeros(nb * BLOCK)
    s[:n] = signs_for(n, seed, epoch)
    blocks = pad.reshape(m, nb, BLOCK)
    with np.errstate(invalid="ignore", over="ignore"):
        return np.stack([blocks.sum(-1), (blocks * s.reshape(nb, BLOCK)).sum(-1), (blocks ** 2).sum(-1),
                         np.abs(blocks).sum(-1)], -1)


def zscores_from_stats(A, B, stats, bias=None, *, z: float = 6.0, nfma=None, seed: int = 1, epoch: int = 0,
                       abs_floor: float = ABS_FLOOR) -> Scores:
    """Every checksum's score (1, m, nb, 2); A (m, k), B (k, n) float32 arrays of 16-bit values, stats (m, nb, 4)
    float64 (fused.py:188-235)."""
    u = ACC_UNIT
    A3, B3 = _f32(A)[None], _f32(B)[None]
    stats = np.asarray(stats, np.float64)
    m, k = A3.shape[-2:]
    n = B3.shape[-1]
    steps = k / nfma if nfma else 0.0
    A_norm = _norm2(A3, -1)[:, :, None]
    A_l1 = np.sum(np.abs(A3), axis=-1, dtype=np.float32)[:, :, None]
    zs_all, den_all, exp_all, act_all, unknown = [], [], [], [], False
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for sp in spans(n, BLOCK):
            start, width, nblk = sp.start, sp.width, sp.nblk
            end = start + width * nblk
            b0 = start // BLOCK
            st = stats[None, :, b0:b0 + nblk]                                   # (1, m, nblk, 4)
            s = _signs(width, seed, epoch)
            Bblk = B3[..., start:end].reshape(1, k, nblk, width)
            B2 = _pair_sums64(Bblk, s)
            expected = np.matmul(A3.astype(np.float64), B2.reshape(1, k, 2 * nblk)).reshape(1, m, nblk, 2)
            bound = (A_l1 * _amax_nan(Bblk, (-3, -1))[:, None, :]).astype(np.float32)
            if bias is not None:
                bb = _f32(bias)[start:end].reshape(nblk, width)
                expected = expected + _pair_sums64(bb, s)
                bound = (bound + _amax_nan(bb, -1)).astype(np.float32)
            actual = st[..., :2]
            cnorm = np.sqrt(np.maximum(st[..., 2], 0.0)).astype(np.float32)     # np.maximum keeps NaN
            l1 = st[..., 3].astype(np.float32)
            b_frob = _norm2(Bblk.transpose(0, 2, 1, 3).reshape(1, nblk, k * width), -1)[:, None, :]
            per_out = ACC_C2 * math.sqrt(k) + ACC_C3 * steps + math.sqrt(width)
            prod = ((A_norm * b_frob) * f32(ACC_C1 * math.sqrt(k) * u)).astype(np.float32)
            prod = np.where(np.isfinite(prod), prod, bound * f32(u * 128)).astype(np.float32)
            noise = (cnorm * f32(per_out * u) + prod).astype(np.float32)[..., None]
            den = (noise + f32(abs_floor)).astype(np.float32).astype(np.float64)
            diff = np.abs(expected - actual)
            zs = diff / den
            worst = ((l1 * f32(per_out * u) + prod)[..., None] + f32(abs_floor)).astype(np.float32)
            zs[..., :1] = np.minimum(zs[..., :1], diff[..., :1] / worst.astype(np.float64) * z)
            zs = _judge_nonfinite(zs.astype(np.float32), expected, actual, noise, bound[..., None], "fp32",
                                  cnorm[..., None], width, 0.0, k)
            unknown = unknown or bool((zs < 0).any())
            zs_all.append(zs)
            den_all.append(np.broadcast_to(den.astype(np.float32), zs.shape))
            exp_all.append(expected)
            act_all.append(np.broadcast_to(actual, zs.shape))
    return _scores(zs_all, den_all, exp_all, act_all, unknown, m, z)


def _scores(zs_all, den_all, exp_all, act_all, unknown, m, z) -> Scores:
    best = None
    for i, zz in enumerate(zs_all):
        flat = zz.reshape(-1)
        j = int(np.argmax(flat))
        if best is None or flat[j] > best[0]:
            best = (float(flat[j]), i, j)
    mz, si, j = best
    nblk_i = zs_all[si].shape[2]
    _, rem = divmod(j // 2, m * nblk_i)
    r_i, c_i = divmod(rem, nblk_i)
    col_block = sum(z_.shape[2] for z_ in zs_all[:si]) + c_i
    noise_at = float(den_all[si].reshape(-1)[j])
    if unknown and mz <= z:                                            # checksum.py:349-356
        mz = -1.0
    Z = np.concatenate(zs_all, axis=2)
    return Scores(z=Z, den=np.concatenate(den_all, axis=2), expected=np.concatenate(exp_all, axis=2),
                  actual=np.concatenate(act_all, axis=2), csb=np.zeros_like(Z), max_z=mz, batch=0, row=r_i,
                  col_block=col_block, noise=noise_at, unknown=unknown)


def pow2_scale(wmax: float) -> float:
    """fused.py:262-270: the power of two that puts 128 * wmax in [2^14, 2^15); 1 when wmax isn't finite."""
    e = (int(np.array([f32(wmax) * f32(128.0)], np.float32).view(np.int32)[0]) >> 23) & 0xFF
    e = 141 if e == 255 else max(e, 15)
    return float(np.array([(e - 14) << 23], np.int32).view(np.float32)[0])


def _round16(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 -> nearest bf16/fp16 value (ties to even), as float32."""
    x = np.asarray(x, np.float32)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(x)
    out = r.view(np.float32).copy()
    out[nan] = np.nan
    return out


def block_sum_parts(B, dtype: str = "bf16", *, seed: int = 1, epoch: int = 0):
    """The W side of the self-check for B (k, n) float32 of 16-bit values (fused.py:272-316): per block j
    parts (k, nb, 6) float32 (hi, mid, lo of the plain block sum, then of the signed one; fp16: of the block sums
    divided by scale[j]), scale (nb,), and aux (nb, 4): sum of W^2, of plain block sums^2, of signed block sums^2, and
    max |W| (NaN as Inf).  The block sums are float64 sums rounded once to fp32."""
    B = _f32(B)
    k, n = B.shape
    nb = -(-n // BLOCK)
    parts = np.zeros((k, nb, 6), np.float32)
    scale = np.ones(nb)
    aux = np.zeros((nb, 4))
    for j in range(nb):
        lo_c, hi_c = j * BLOCK, min(n, (j + 1) * BLOCK)
        s = _signs(hi_c - lo_c, seed, epoch).astype(np.float64)
        blk = B[:, lo_c:hi_c].astype(np.float64)
        bp = blk.sum(1).astype(np.float32)
        bs = (blk * s).sum(1).astype(np.float32)
        with np.errstate(invalid="ignore", over="ignore"):
            aux[j] = [(blk ** 2).sum(), (bp.astype(np.float64) ** 2).sum(), (bs.astype(np.float64) ** 2).sum(),
                      float(np.max(np.where(np.isnan(blk), np.inf, np.abs(blk)))) if k else 0.0]
        if dtype == "fp16":
            scale[j] = pow2_scale(float(np.float32(aux[j, 3])))
        for q, x in enumerate((bp, bs)):
            xs = (x / f32(scale[j])).astype(np.float32)
            hi = _round16(xs, dtype)
            r = (xs - hi).astype(np.float32)
            mid = _round16(r, dtype)
            lo = _round16((r - mid).astype(np.float32), dtype)
            parts[:, j, 3 * q:3 * q + 3] = np.stack([hi, mid, lo], 1)
    return parts, scale, aux


def checked_scores(A, B, stats, bias=None, *, dtype: str = "bf16", z: float = 6.0, nfma=None, seed: int = 1,
                   epoch: int = 0, abs_floor: float = ABS_FLOOR, expected=None):
    """The self-check's scores (m, nb, 2) float32 and noise (m, nb) of C = A @ B + bias (fused.py:419-458), with the
    accumulator's block statistics `stats` (m, nb, 4) as the actual side, and the expected sides (m, nb, 2) given,
    or computed as A . (block sums of B), block sums rounded once to fp32, in float64 (plus the bias's block sums).
    Returns (z, den, expected)."""
    u = f32(ACC_UNIT)
    A = _f32(A)
    B = _f32(B)
    m, k = A.shape
    n = B.shape[1]
    nb = -(-n // BLOCK)
    stats = np.asarray(stats, np.float64)
    parts, scale, aux = block_sum_parts(B, dtype, seed=seed, epoch=epoch)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        if expected is None:
            sums = (parts[:, :, 0:3].astype(np.float64).sum(-1), parts[:, :, 3:6].astype(np.float64).sum(-1))
            expected = np.stack([A.astype(np.float64) @ (s_ * scale[None, :]) for s_ in sums], -1)    # (m, nb, 2)
            if bias is not None:
                bsum = np.zeros((nb, 2))
                for j in range(nb):
                    lo_c, hi_c = j * BLOCK, min(n, (j + 1) * BLOCK)
                    bsum[j] = _pair_sums64(_f32(bias)[lo_c:hi_c], _signs(hi_c - lo_c, seed, epoch))
                expected = expected + bsum[None]
        expected = np.asarray(expected, np.float64)
        an = np.sqrt((A.astype(np.float64) ** 2).sum(1)).astype(np.float32)[:, None]
        al1 = np.abs(A.astype(np.float64)).sum(1).astype(np.float32)[:, None]
        bound_b = np.zeros(nb, np.float32)
        if bias is not None:
            for j in range(nb):
                bound_b[j] = _amax_nan(_f32(bias)[j * BLOCK:min(n, (j + 1) * BLOCK)], -1)
        width = np.array([min(BLOCK, n - j * BLOCK) for j in range(nb)], np.float32)[None, :]
        kf = f32(k)
        sk = np.sqrt(kf)
        steps = f32(k / nfma if nfma else 0.0)
        per_out = (f32(ACC_C2) * sk + f32(ACC_C3) * steps + np.sqrt(width)).astype(np.float32)
        bfro2, bsp2, bss2, bmax = (aux[:, q].astype(np.float32)[None, :] for q in range(4))
        bound = (al1 * bmax + bound_b[None, :]).astype(np.float32)
        stand = (bound * (u * f32(128.0))).astype(np.float32)
        prod = (an * np.sqrt(bfro2) * (f32(ACC_C1) * sk * u)).astype(np.float32)
        prod = np.where(np.isfinite(prod), prod, stand).astype(np.float32)
        cn = np.sqrt(np.maximum(stats[..., 2], 0.0)).astype(np.float32)
        cl1 = stats[..., 3].astype(np.float32)
        noise = (cn * (per_out * u) + prod).astype(np.float32)
        skc = np.sqrt(f32(min(k, 32)))
        e32 = expected.astype(np.float32)
        ex = [(an * np.sqrt(q2) * (f32(ACC_C1) * skc * u) + f32(4.0) * u * np.abs(e32[..., i])).astype(np.float32)
              for i, q2 in enumerate((bsp2, bss2))]
        ex = [np.where(np.isfinite(e), e, stand).astype(np.float32) for e in ex]
        noise_ps = [(noise + e).astype(np.float32) for e in ex]
        dens = [(npn + f32(abs_floor)).astype(np.float32) for npn in noise_ps]
        act = stats[..., :2]
        d = np.abs(expected - act)
        zp = (d[..., 0] / dens[0].astype(np.float64)).astype(np.float32)
        zs = (d[..., 1] / dens[1].astype(np.float64)).astype(np.float32)
        worst = (cl1 * (per_out * u) + prod + ex[0] + f32(abs_floor)).astype(np.float32)
        zw = (d[..., 0] / worst.astype(np.float64) * z).astype(np.float32)
        zp = np.minimum(zp, zw)                                              # NaN in either stays NaN
        lim = (bound * f32(1.01)).astype(np.float32)
        e_bad = ~(np.abs(e32[..., 0]) < np.inf) | ~(np.abs(e32[..., 1]) < np.inf)
        a32 = act.astype(np.float32)
        a_bad = (~(np.abs(a32[..., 0]) < np.inf) | ~(np.abs(a32[..., 1]) < np.inf)) & ~e_bad
        n_bad = (~(noise_ps[0] < np.inf) | ~(noise_ps[1] < np.inf)) & ~e_bad & ~a_bad
        cap = (bound * (f32(1.02) + kf * f32(2.0 ** -22))).astype(np.float32)
        imposs = ~e_bad & ~a_bad & ~n_bad & (lim < BIG) & (cn > cap * np.sqrt(width))
        for_bad = np.where(lim < min(F32_MAX, BIG), f32(np.inf), f32(-1.0))
        out = []
        for zz in (zp, zs):
            zz = np.where(zz == zz, zz, f32(-1.0))
            zz = np.where(imposs, f32(np.inf), zz)
            zz = np.where(a_bad | n_bad, for_bad, zz)
            zz = np.where(e_bad, f32(-1.0), zz)
            out.append(zz.astype(np.float32))
        Z = np.stack(out, -1)
        den = np.where(Z[..., 0] >= Z[..., 1], dens[0], dens[1]).astype(np.float32)
    return Z, den, expected
