"""Precise (fp32-accumulator) column-block check of C = beta*bias + alpha*(A @ B) (oracle: test infrastructure only).

Restates checksum.py:537-692 (`matmul_zscores_acc`, `_acc_zscores`, `check_matmul_acc`) in numpy: A and B hold
bf16/fp16 values, C is the fp32 product itself (not rounded to 16 bits).  Both sides of every checksum are float64
(block sums of B and of C, A @ B2), and the noise is the fp32 accumulation's rounding of the result alone:

    u (C1 sqrt(k) |alpha| |a_row|_2 |B_block|_F + (C2 sqrt(k) + C3 k / nfma + sqrt(width)) |C_block|_2),  u = 2^-24

with the Inf/NaN rules of `_judge_nonfinite` (float32 outputs, no subnormal step) and `_complete_score`.  Norms,
bounds and the noise are float32 in the reference's order of operations; ``acc_zscores`` returns every checksum's
score (the reference keeps the worst), ties resolved as torch.max on the CPU does (first in row-major order).
"""
from __future__ import annotations

import math

import numpy as np

from .abft import UNJUDGED, Scores, _amax_nan, _f32, _judge_nonfinite, _norm1, _norm2, spans
from .lowp import ABS_FLOOR
from .signs import signs as _signs

ACC_UNIT = 2.0 ** -24                       # checksum.py:558
ACC_C1, ACC_C2, ACC_C3 = 0.6, 1.0, 1.0      # checksum.py:559
f32 = np.float32


def _pair_sums64(xb, s) -> np.ndarray:
    """(..., width) -> (..., 2) float64 plain and signed sums (checksum.py:566-575)."""
    x = np.asarray(xb, np.float64)
    return np.stack([x.sum(-1), (x * s.astype(np.float64)).sum(-1)], axis=-1)


def acc_zscores(A, B, C, bias=None, *, alpha: float = 1.0, beta: float = 1.0, block: int = 128,
                abs_floor: float = ABS_FLOOR, z: float = 6.0, nfma=None, seed: int = 1, epoch: int = 0) -> Scores:
    """Every checksum's score; A (m,k)|(bA,m,k), B (k,n)|(bB,k,n) float32 arrays of 16-bit values, C (m,n)|(b,m,n)
    float32 (checksum.py:599-686)."""
    u = ACC_UNIT
    A3, B3, C3 = (_f32(t) if _f32(t).ndim == 3 else _f32(t)[None] for t in (A, B, C))
    nb_batch, m, n = C3.shape
    k = A3.shape[-1]
    if k == 0:                                         # checksum.py:386-392: one zero column
        A3 = np.zeros(A3.shape[:-1] + (1,), np.float32)
        B3 = np.zeros(B3.shape[:-2] + (1, n), np.float32)
        k = 1
    steps = k / nfma if nfma else 0.0
    nbt = max(nb_batch, A3.shape[0], B3.shape[0])
    A_norm = _norm2(A3, -1)[:, :, None]                              # (bA, m, 1)
    A_l1 = _norm1(A3, -1)[:, :, None]
    zs_all, den_all, exp_all, act_all, unknown = [], [], [], [], False
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for sp in spans(n, block):
            start, width, nblk = sp.start, sp.width, sp.nblk
            end = start + width * nblk
            s = _signs(width, seed, epoch)
            Cb = C3[..., start:end].reshape(nb_batch, m, nblk, width)
            Bblk = B3[..., start:end].reshape(B3.shape[0], k, nblk, width)
            B2 = _pair_sums64(Bblk, s)                                   # (bB, k, nblk, 2)
            expected = np.matmul(A3.astype(np.float64), B2.reshape(B3.shape[0], k, 2 * nblk)).reshape(-1, m, nblk, 2)
            bound = (A_l1 * _amax_nan(Bblk, (-3, -1))[:, None, :]).astype(np.float32)      # (b, m, nblk)
            if alpha != 1.0:
                expected = expected * alpha
                bound = (bound * f32(abs(alpha))).astype(np.float32)
            if bias is not None and beta != 0:
                bias_ = _f32(bias)
                if bias_.ndim == 1:
                    bb = np.broadcast_to(bias_, (n,))[start:end].reshape(nblk, width)
                elif bias_.ndim <= 2:
                    bb = np.broadcast_to(bias_, (m, n))[:, start:end].reshape(m, nblk, width)
                else:
                    bb = np.broadcast_to(bias_, (nb_batch, m, n))[..., start:end].reshape(nb_batch, m, nblk, width)
                expected = expected + beta * _pair_sums64(bb, s)
                bound = (bound + f32(abs(beta)) * _amax_nan(bb, -1)).astype(np.float32)
            actual = _pair_sums64(Cb, s)                                 # (b, m, nblk, 2)
            cnorm = _norm2(Cb, -1)                                       # (b, m, nblk)
            b_frob = _norm2(Bblk.reshape(B3.shape[0], k, nblk, width).transpose(0, 2, 1, 3).reshape(
                B3.shape[0], nblk, k * width), -1)[:, None, :]           # (bB, 1, nblk)
            per_out = ACC_C2 * math.sqrt(k) + ACC_C3 * steps + math.sqrt(width)
            prod = ((A_norm * b_frob) * f32(ACC_C1 * math.sqrt(k) * abs(alpha) * u)).astype(np.float32)
            prod = np.where(np.isfinite(prod), prod, bound * f32(u * 128)).astype(np.float32)
            noise = (cnorm * f32(per_out * u) + prod).astype(np.float32)[..., None]        # (b, m, nblk, 1)
            den = (noise + f32(abs_floor)).astype(np.float32).astype(np.float64)
            diff = np.abs(expected - actual)
            zs = diff / den
            worst = ((_norm1(Cb, -1) * f32(per_out * u) + prod)[..., None] + f32(abs_floor)).astype(np.float32)
            zs[..., :1] = np.minimum(zs[..., :1], diff[..., :1] / worst.astype(np.float64) * z)
            zs = _judge_nonfinite(zs.astype(np.float32), expected, actual, noise, bound[..., None], "fp32",
                                  cnorm[..., None], width, 0.0, k)
            unknown = unknown or bool((zs < 0).any())
            zs_all.append(np.broadcast_to(zs, (nbt, m, nblk, 2)))
            den_all.append(np.broadcast_to(den.astype(np.float32), (nbt, m, nblk, 2)))
            exp_all.append(np.broadcast_to(expected, (nbt, m, nblk, 2)))
            act_all.append(np.broadcast_to(actual, (nbt, m, nblk, 2)))
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
    Z = np.concatenate(zs_all, axis=2)
    return Scores(z=Z, den=np.concatenate(den_all, axis=2), expected=np.concatenate(exp_all, axis=2),
                  actual=np.concatenate(act_all, axis=2), csb=np.zeros_like(Z), max_z=mz, batch=b_i, row=r_i,
                  col_block=col_block, noise=noise_at, unknown=unknown)
