"""The oracle against the reference's own answers on seeded cases (tests/golden/*.npz, written by
tests/golden/make_golden.py from the reference's checksum.py / serve.py).

Scores are compared checksum by checksum.  The reference computes the expected side with an fp32 GEMM (whose
rounding depends on the BLAS) and the oracle in float64 rounded once, so scores may differ by that GEMM's
rounding in noise units plus 1e-3 relative:
    |dz| <= 1e-3 * max(1, z) + 2^-22 * |a_row|_2 |checksum column|_2 / noise
(four fp32 ulps of the Cauchy-Schwarz bound of the GEMM's partial sums).
Special scores (inf, the unjudged -1 / 0) must match exactly, as must the location of every fault and every
verdict.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import abft, serve_check, signs
from tests import _golden as G

TRAIN = G.load("train.npz")
SERVE = G.load("serve.npz")


def _shape(row):
    return tuple(int(v) for v in row if v)


def gemm_slack(csb, den) -> np.ndarray:
    """The fp32 expected side's rounding, in noise units: 4 ulps of |a_row|_2 |checksum column|_2 / noise."""
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        s = 2.0 ** -22 * np.asarray(csb, np.float64) / np.asarray(den, np.float64)
    return np.where(np.isfinite(s), s, 0.0)


def z_close(ours: np.ndarray, ref: np.ndarray, slack=0.0) -> np.ndarray:
    ours, ref = np.asarray(ours, np.float64), np.asarray(ref, np.float64)
    both_inf = np.isinf(ours) & np.isinf(ref)
    fin = np.isfinite(ours) & np.isfinite(ref)
    tol = 1e-3 * np.maximum(1.0, np.abs(ref)) + slack
    with np.errstate(invalid="ignore"):
        ok = both_inf | (fin & (np.abs(ours - ref) <= tol))
    special = (ref < 0) | (ref == 0)
    with np.errstate(invalid="ignore"):
        ok &= ~special | (ours == ref) | (fin & (np.abs(ours - ref) <= 1e-3 + slack))
    return ok


def test_sign_tables_match_reference():
    s = G.load("signs.npz")
    seed = int(s["seed"])
    assert np.array_equal(signs.sign_table(seed, 0), s["epoch0"])
    assert np.array_equal(signs.sign_table(seed, 3), s["epoch3"])


def train_case(i):
    p = f"c{i}_"
    ids = [str(v) for v in TRAIN[p + "ids"]]
    shp = TRAIN[p + "shapes"]
    alpha, beta, is16 = TRAIN[p + "meta"]
    dt = "fp16" if is16 else "bf16"
    A = G.as_f32(G.words(TRAIN, ids[0]), dt).reshape(_shape(shp[0]))
    B = G.as_f32(G.words(TRAIN, ids[1]), dt).reshape(_shape(shp[1]))
    C = G.as_f32(G.words(TRAIN, ids[2]), dt).reshape(_shape(shp[2]))
    bias = G.as_f32(G.words(TRAIN, ids[3]), dt).reshape(_shape(shp[3])) if ids[3] else None
    return A, B, C, bias, float(alpha), float(beta), dt


@pytest.mark.parametrize("i", range(len(G.names(TRAIN))))
def test_training_check_matches_reference(i):
    name = G.names(TRAIN)[i]
    A, B, C, bias, alpha, beta, dt = train_case(i)
    s = abft.zscores(A, B, C, bias, alpha=alpha, beta=beta, dtype=dt, seed=1)
    n = C.shape[-1]
    nbf = n // min(128, n)
    def flat(a):
        return np.concatenate([a[:, :, :nbf].reshape(-1), a[:, :, nbf:].reshape(-1)])
    ours = flat(s.z)
    ref = TRAIN[f"c{i}_zs"]
    assert ours.shape == ref.shape, name
    ok = z_close(ours, ref, flat(gemm_slack(s.csb, s.den)))
    assert ok.all(), (name, np.nonzero(~ok)[0][:5], ours[~ok][:5], ref[~ok][:5])
    mz, b, r, blk, noise = TRAIN[f"c{i}_result"]
    assert (s.max_z > 6) == (mz > 6) and ((s.max_z < 0) == (mz < 0)), (name, s.max_z, mz)
    if mz > 6 or mz < 0:
        assert math.isinf(s.max_z) == math.isinf(mz) and (mz < 0 or math.isinf(mz) or abs(s.max_z - mz) <= 1e-3 * mz)
    if mz > 6:
        assert (s.row, s.col_block) == (int(r), int(blk)), name
        if C.ndim == 3:
            assert s.batch == int(b)


def serve_case(i):
    p = f"c{i}_"
    ids = [str(v) for v in SERVE[p + "ids"]]
    m, k, n = (int(v) for v in SERVE[p + "shape"])
    dt = "fp16" if int(SERVE[p + "dtype"]) else "bf16"
    x = G.as_f32(G.words(SERVE, ids[0]), dt).reshape(m, k)
    W = G.as_f32(G.words(SERVE, ids[1]), dt).reshape(n, k)
    y = G.as_f32(G.words(SERVE, ids[2]), dt).reshape(m, n)
    b = G.as_f32(G.words(SERVE, ids[3]), dt).reshape(n) if ids[3] else None
    return x, W, b, y, dt


@pytest.mark.parametrize("i", range(len(G.names(SERVE))))
def test_serving_check_matches_reference(i):
    name = G.names(SERVE)[i]
    x, W, b, y, dt = serve_case(i)
    c = serve_check.layer_constants(W, b, 128, dt, seed=1)
    s = serve_check.check_static(x, y, c, dtype=dt, seed=1)
    ref = SERVE[f"c{i}_zs"]
    ours = s.z.reshape(-1)
    ok = z_close(ours, ref, gemm_slack(s.csb, s.den).reshape(-1))
    assert ok.all(), (name, np.nonzero(~ok)[0][:5], ours[~ok][:5], ref[~ok][:5])
    st = SERVE[f"c{i}_state"]
    assert int(s.state[2]) == int(st[2]) and int(s.state[3]) == int(st[3]), (name, s.state, st)
    rz, rf, _ = serve_check.decode(st[0], st[1])
    oz, of, _ = serve_check.decode(s.state[0], s.state[1])
    assert (oz > 6) == (rz > 6), (name, oz, rz)
    if rz > 6:
        assert of // 2 == rf // 2, (name, of, rf)
