"""The torch CPU restatement (oracle.torch_check, the benchmark's CPU baseline) against the numpy oracle, which the
reference's golden vectors pin: scores within fp32 rounding of the expected side, identical verdicts and locations,
on clean, faulted, biased, ragged and non-finite problems."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import abft, torch_check
from oracle.lowp import bf16_round


def _problem(m, k, n, seed, bias):
    r = np.random.default_rng(seed)
    A = bf16_round(r.standard_normal((m, k)).astype(np.float32))
    B = bf16_round((r.standard_normal((k, n)) * 0.05).astype(np.float32))
    b = bf16_round((r.standard_normal(n) * 0.1).astype(np.float32)) if bias else None
    C = A.astype(np.float64) @ B.astype(np.float64)
    if b is not None:
        C = C + b
    return A, B, b, bf16_round(C.astype(np.float32))


@pytest.mark.parametrize("m,k,n,bias,fault", [(64, 256, 384, False, None), (33, 130, 300, True, None),
                                              (64, 256, 384, False, (5, 200, 0.5)),
                                              (48, 512, 256, True, (47, 255, 16.0)),
                                              (16, 64, 128, False, (3, 7, np.inf)),
                                              (16, 64, 130, False, (2, 129, np.nan))])
def test_matches_numpy_oracle(m, k, n, bias, fault):
    A, B, b, C = _problem(m, k, n, seed=m + k + n, bias=bias)
    if fault is not None:
        i, j, d = fault
        C[i, j] = C[i, j] + d if np.isfinite(d) else d
    want = abft.zscores(A, B, C, b)
    T = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a))   # noqa: E731
    Z, worst, (row, blk) = torch_check.zscores(T(A), T(B), T(C), T(b))
    Z = Z.numpy()
    zw = want.z[0]
    fin = np.isfinite(zw)
    assert np.array_equal(fin, np.isfinite(Z))
    assert np.array_equal(zw[~fin], Z[~fin])
    # the expected sides differ by fp32 GEMM rounding (float64 in the numpy oracle): relative to the noise
    slack = want.csb[0][fin] * 2.0 ** -20 / want.den[0][fin]
    assert (np.abs(Z[fin] - zw[fin]) <= 1e-4 * np.abs(zw[fin]) + slack + 1e-6).all()
    assert ((Z > 6) == (zw > 6)).all()
    if fault is not None:
        assert (row, blk) == (want.row, want.col_block)
        assert (worst > 6) == (want.max_z > 6) and (np.isfinite(worst) == np.isfinite(want.max_z))


def test_linear_both_is_column_check_and_row_check_of_the_transpose():
    A, B, b, C = _problem(256, 128, 256, seed=5, bias=True)
    C[200, 17] += 1.0
    x, W, y = torch.from_numpy(A), torch.from_numpy(np.ascontiguousarray(B.T)), torch.from_numpy(C)
    (zc, wc, lc), (zr, wr, lr) = torch_check.linear_both(x, W, torch.from_numpy(b), y)
    assert zc.shape == (256, 2, 2) and zr.shape == (256, 2, 2)
    assert lc == (200, 0) and lr == (17, 1) and wc > 6 and wr > 6
    want = abft.zscores(B.T, A.T, C.T, b[:, None])
    assert (want.row, want.col_block) == lr
    assert np.allclose(zr.numpy(), want.z[0], rtol=1e-3, atol=1e-3)
