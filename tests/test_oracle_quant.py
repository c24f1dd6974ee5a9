"""The quantized-GEMM checks of the oracle (oracle/quant.py) pinned to the reference's modes.judge (golden vectors,
tests/golden/quant.npz), to its own known-answer test (tests/test_modes.py:47-64 of the reference: every input at
+-127) and to brute force; the scaled fp8 identity (no reference function) to exact invariants."""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle import quant
from tests import _golden as G

Q = G.load("quant.npz")
NCASES = sum(1 for k in Q.files if k.endswith("_nf"))


def _case(i, f):
    a, b, c = Q[f"q{i}_a"], Q[f"q{i}_b"], Q[f"q{i}_c"].copy()
    r, j = (int(v) for v in Q[f"q{i}_f{f}_at"])
    c[r, j] = Q[f"q{i}_f{f}_v"]
    return str(Q[f"q{i}_name"]), a, b, c, Q[f"q{i}_f{f}_z"], int(Q[f"q{i}_f{f}_wrong"])


def _cases(mode):
    for i in range(NCASES):
        if str(Q[f"q{i}_name"]).startswith(mode):
            for f in range(int(Q[f"q{i}_nf"])):
                yield i, f


def test_e4m3_table_matches_torch():
    vals = quant.fp8_e4m3_values()
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    same = (vals == t) | (np.isnan(vals) & np.isnan(t))
    assert same.all()


@pytest.mark.parametrize("i,f", list(_cases("int8")))
def test_int8_matches_reference(i, f):
    name, a, b, c, z, wrong = _case(i, f)
    res = quant.int8_judge(a, b, c, quant.patterns(1))
    assert res["wrong_blocks"] == wrong, name
    assert np.array_equal(res["bad"], np.isinf(z)), name


@pytest.mark.parametrize("i,f", list(_cases("fp8")))
def test_fp8_unit_scales_match_reference(i, f):
    """With sa = sb = 1 and an fp32 result the scaled check is modes.judge('fp8', nfma=16, unit=2^-14)."""
    name, a, b, c, z, wrong = _case(i, f)
    vals = quant.fp8_e4m3_values()
    A, B = vals[a], vals[b]
    res = quant.fp8_judge(A, B, np.ones(A.shape[0]), np.ones(B.shape[1]), c.astype(np.float64), quant.patterns(1))
    assert res["wrong_blocks"] == wrong, name
    fin = np.isfinite(z)
    assert np.array_equal(np.isinf(res["z"]), ~fin), name
    assert np.allclose(res["z"][fin], z[fin], rtol=1e-5, atol=1e-6), name


def test_int8_known_answer_at_the_largest_values():
    """Reference test_modes.py:47-64: every input +-127 at k = 1024; outputs of +-16,516,096; one output off by 1
    is one wrong block."""
    a = np.full((64, 1024), 127, np.int8)
    b = np.full((1024, 256), 127, np.int8)
    b[:, ::3] = -127
    c = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32)
    assert int(np.abs(c).min()) == 127 * 127 * 1024 == 16516096
    W = quant.patterns(1)
    assert quant.int8_judge(a, b, c, W)["wrong_blocks"] == 0
    c[5, 200] += 1
    res = quant.int8_judge(a, b, c, W)
    assert res["wrong_blocks"] == 1 and res["bad"][5, 1]


def test_int8_sums_brute_force():
    rng = np.random.default_rng(3)
    m, k, n = 3, 7, 300                               # a narrower last block of 44
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    c = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32)
    W = quant.patterns(1)
    actual, expected = quant.int8_sums(a, b, c, W)
    W44 = quant.patterns(1, 44)                      # the last block's own pattern
    for i, blk, p in itertools.product(range(m), range(3), range(2)):
        lo, hi = 128 * blk, min(128 * blk + 128, n)
        w = [int((W if hi - lo == 128 else W44)[p, j - lo]) for j in range(lo, hi)]
        act = sum(int(c[i, j]) * w[j - lo] for j in range(lo, hi))
        exp = sum(int(a[i, kk]) * sum(int(b[kk, j]) * w[j - lo] for j in range(lo, hi)) for kk in range(k))
        assert actual[i, blk, p] == act and expected[i, blk, p] == exp


def _fp8_problem(seed, m=12, k=256, n=384):
    """Quantized inputs with per-row / per-column scales 10^U(-3,-1), the fp32 result of the scaled product."""
    rng = np.random.default_rng(seed)
    vals = quant.fp8_e4m3_values()
    finite = np.nonzero(np.isfinite(vals) & (np.abs(vals) >= 2.0 ** -6) | (vals == 0))[0]
    aq = rng.choice(finite, (m, k)).astype(np.uint8)
    bq = rng.choice(finite, (k, n)).astype(np.uint8)
    A, B = vals[aq], vals[bq]
    sa = 10.0 ** rng.uniform(-3, -1, m)
    sb = 10.0 ** rng.uniform(-3, -1, n)
    C = ((sa[:, None] * (A @ B)) * sb[None, :]).astype(np.float32)
    return A, B, sa, sb, C


def test_fp8_scaled_identity_brute_force():
    """The expected side sa_i Aq_i . (sum_j w_j sb_j Bq_j) equals the checksum of the exact scaled product."""
    A, B, sa, sb, _ = _fp8_problem(1, m=2, k=5, n=130)
    W = quant.patterns(1)
    exact = (sa[:, None] * (A @ B)) * sb[None, :]
    res = quant.fp8_judge(A, B, sa, sb, exact, W)
    assert res["wrong_blocks"] == 0 and res["worst_z"] < 1e-6


def test_fp8_scale_invariance():
    """Scaling row i's activation scale and its outputs, or a block's weight scales and its outputs, by the same
    power of two changes no z (exactly); a z that used an unscaled norm or expected side would move."""
    A, B, sa, sb, C = _fp8_problem(2)
    W = quant.patterns(1)
    z0 = quant.fp8_judge(A, B, sa, sb, C, W)["z"]
    f = 2.0 ** np.arange(-3, 9)[:, None]
    z1 = quant.fp8_judge(A, B, sa * f[:, 0], sb, C.astype(np.float64) * f, W)["z"]
    assert np.array_equal(z0, z1)
    g = 2.0 ** np.repeat(np.array([-2, 3, 1]), 128)[None, :]        # one power of two per block of columns
    z2 = quant.fp8_judge(A, B, sa, sb * g[0], C.astype(np.float64) * g, W)["z"]
    assert np.array_equal(z0, z2)


def test_fp8_scaled_faults():
    """Clean scaled results stay far below the alarm; a fault of half a typical output, NaN, and an impossible
    value are each one wrong block at their (row, block)."""
    A, B, sa, sb, C = _fp8_problem(3)
    W = quant.patterns(1)
    res = quant.fp8_judge(A, B, sa, sb, C, W)
    assert res["wrong_blocks"] == 0 and res["worst_z"] < 1.0
    for r, j, kind in [(4, 300, "add"), (0, 5, "nan"), (11, 130, "huge")]:
        c = C.astype(np.float64).copy()
        blk = c[r, (j // 128) * 128:(j // 128 + 1) * 128]
        c[r, j] = {"add": c[r, j] + 0.5 * np.sqrt((blk ** 2).mean()), "nan": np.nan, "huge": 1e30}[kind]
        z = quant.fp8_judge(A, B, sa, sb, c, W)["z"]
        assert (z > 6).sum() == 1 and z[r, j // 128] > 6, kind


def test_fp8_bf16_output_adds_its_rounding():
    """A bf16 result: its rounding (half a unit in the last place: between 2^-9 and 2^-8 of the output, by where it
    sits in its binade) is priced by the added 2^-8 |C_blk| term -- the unit the reference's serving check gives
    bf16 outputs -- and lowers every z."""
    A, B, sa, sb, C = _fp8_problem(4)
    c16 = torch.from_numpy(C).bfloat16().float().numpy().astype(np.float64)
    W = quant.patterns(1)
    z0 = quant.fp8_judge(A, B, sa, sb, c16, W)["z"]
    res = quant.fp8_judge(A, B, sa, sb, c16, W, c_bf16=True)
    assert res["wrong_blocks"] == 0 and res["worst_z"] < 1.0 and (res["z"] < z0).all()


def worst_rounding_problem():
    """Rows whose 128 outputs of a block all round the same way by the most bf16 allows: C = sa_i (1 x 1 fp8 ones),
    sa_i chosen so the exact output sits just below / above a rounding midpoint.  Row 0: just below 2 - 2^-8 (rounds
    down by 2^-8 - 2^-20: 2^-9 of the value), row 1: just above it (rounds up to 2: 2^-9), row 2: just below
    1 + 2^-8 (rounds down to 1: 2^-8 of the value), row 3: 1.5 (exact).  Returns fp8 values, scales, the exact C and
    its bf16 rounding (float64)."""
    m, n = 4, 256
    v = np.array([2 - 2.0 ** -8 - 2.0 ** -20, 2 - 2.0 ** -8 + 2.0 ** -20, 1 + 2.0 ** -8 - 2.0 ** -20, 1.5])
    A, B = np.ones((m, 1)), np.ones((1, n))
    sa, sb = v.astype(np.float32).astype(np.float64), np.ones(n)
    exact = np.repeat(sa[:, None], n, axis=1)
    c16 = torch.from_numpy(exact).bfloat16().double().numpy()
    return A, B, sa, sb, exact, c16


def test_fp8_bf16_output_term_worst_case():
    """The bf16-output term against its worst case: every output of a block rounded the same way by 2^-9 of its
    value scores sqrt(128) / 2 = 5.66 units less the other noise terms' share and the rounded output's larger norm
    (here 3% at most): in (5.4, 5.66], below the threshold.  By 2^-8 of the value (just above a power of two) the same construction scores about 11: the term
    is a unit-roundoff noise model, as the reference's u = 2^-8 for bf16 outputs, not a worst-case bound.  A term of
    2^-9, or none, would score the first rows 11.2 and about 90; one of 2^-7 would score them 2.8."""
    A, B, sa, sb, exact, c16 = worst_rounding_problem()
    W = quant.patterns(1)
    res = quant.fp8_judge(A, B, sa, sb, c16, W, c_bf16=True)
    z = res["z"]
    assert (5.4 < z[0]).all() and (z[0] <= np.sqrt(128) / 2).all(), z[0]
    assert (5.4 < z[1]).all() and (z[1] <= np.sqrt(128) / 2).all(), z[1]
    assert (z[2] > 10.5).all() and (z[2] < np.sqrt(128)).all(), z[2]
    assert (z[3] == 0).all()
    # the exact outputs score (near) zero: what the rows score is their rounding alone
    assert quant.fp8_judge(A, B, sa, sb, exact, W, c_bf16=True)["worst_z"] < 1e-3
