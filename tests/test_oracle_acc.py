"""The precise-check oracle (oracle/acc.py) against the reference's own answers (tests/golden/acc.npz, written by
tests/golden/make_golden.py from checksum.matmul_zscores_acc / resolve).

Both sides of every checksum are float64 in the reference and in the oracle, and the noise's norms are fp32
reductions whose order differs (torch against numpy): scores agree to 1e-3 relative (with 1e-3 absolute around 0),
special scores (inf, unjudged -1) exactly, and every verdict and fault location exactly.  A planted mistake in the
oracle fails these: a dropped sqrt(k) or nfma term moves every clean score by far more than 1e-3.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import acc
from tests import _golden as G
from tests.test_oracle_golden import _shape, z_close

ACC = G.load("acc.npz")


def acc_case(i):
    p = f"c{i}_"
    ids = [str(v) for v in ACC[p + "ids"]]
    shp = ACC[p + "shapes"]
    alpha, beta, is16, nfma, epoch = ACC[p + "meta"]
    dt = "fp16" if is16 else "bf16"
    def shape(row):
        return tuple(int(v) for v in row[:max(1, int(np.count_nonzero(row)) or 1)]) if np.count_nonzero(row) else ()
    A = G.as_f32(G.words(ACC, ids[0]), dt).reshape(_dims(shp[0], G.words(ACC, ids[0]).size))
    B = G.as_f32(G.words(ACC, ids[1]), dt).reshape(_dims(shp[1], G.words(ACC, ids[1]).size))
    C = G.f32_words(G.words(ACC, ids[2])).reshape(_dims(shp[2], G.words(ACC, ids[2]).size // 2))
    bias = G.as_f32(G.words(ACC, ids[3]), dt).reshape(_shape(shp[3])) if ids[3] else None
    return A, B, C, bias, float(alpha), float(beta), dt, int(nfma) or None, int(epoch)


def _dims(row, size):
    """A stored shape (zero-padded to 3 dims; a dimension may itself be 0, as k = 0)."""
    d = [int(v) for v in row]
    while len(d) > 2 and d[-1] == 0 and np.prod([x for x in d[:-1]]) == size:
        d = d[:-1]
    return tuple(d)


def flat_spans(z, n):
    nbf = n // min(128, n)
    return np.concatenate([z[:, :, :nbf].reshape(-1), z[:, :, nbf:].reshape(-1)])


@pytest.mark.parametrize("i", range(len(G.names(ACC))))
def test_precise_check_matches_reference(i):
    name = G.names(ACC)[i]
    A, B, C, bias, alpha, beta, dt, nfma, epoch = acc_case(i)
    s = acc.acc_zscores(A, B, C, bias, alpha=alpha, beta=beta, nfma=nfma, seed=1, epoch=epoch)
    ours = flat_spans(s.z, C.shape[-1])
    ref = ACC[f"c{i}_zs"]
    assert ours.shape == ref.shape, name
    ok = z_close(ours, ref)
    assert ok.all(), (name, np.nonzero(~ok)[0][:5], ours[~ok][:5], ref[~ok][:5])
    fin = np.isfinite(ours) & np.isfinite(ref) & (ref > 0)
    dz = float(np.max(np.abs(ours[fin] - ref[fin]) / np.maximum(1.0, ref[fin]))) if fin.any() else 0.0
    print(f"{name}: max relative |dz| {dz:.2e} over {int(fin.sum())} checksums")
    mz, b, r, blk, _ = ACC[f"c{i}_result"]
    assert (s.max_z > 6) == (mz > 6) and ((s.max_z < 0) == (mz < 0)), (name, s.max_z, mz)
    if mz > 6:
        assert math.isinf(s.max_z) == math.isinf(mz)
        assert (s.row, s.col_block) == (int(r), int(blk)), name
        if C.ndim == 3:
            assert s.batch == int(b)


def test_clean_precise_scores_are_small_and_faults_large():
    names = G.names(ACC)
    res = {n: ACC[f"c{i}_result"][0] for i, n in enumerate(names)}
    for n, mz in res.items():
        if "clean" in n or n in ("bf16_bmm", "bf16_shared_b", "bf16_epoch3", "bf16_k2048", "bf16_bias_mat",
                                 "bf16_bias_vec_alpha_beta", "bf16_remainder_300", "bf16_tiny_0", "bf16_tiny_1e-24",
                                 "bf16_k0"):
            assert 0 <= mz <= 6, (n, mz)
    for n in ("bf16_rel_2e-10", "bf16_remainder_fault", "bf16_plus1"):
        assert res[n] > 6, (n, res[n])
    for n in ("bf16_nan", "bf16_inf", "bf16_huge_cancel"):
        assert math.isinf(res[n]), (n, res[n])
    assert res["bf16_nan_row_unjudged"] == -1.0
