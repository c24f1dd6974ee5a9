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
    """A bf16 result: its rounding (at most 2^-9 per output) is priced by the added 2^-8 |C_blk| term -- the unit
    the reference's serving check gives bf16 outputs -- and lowers every z."""
    A, B, sa, sb, C = _fp8_problem(4)
    c16 = torch.from_numpy(C).bfloat16().float().numpy().astype(np.float64)
    W = quant.patterns(1)
    z0 = quant.fp8_judge(A, B, sa, sb, c16, W)["z"]
    res = quant.fp8_judge(A, B, sa, sb, c16, W, c_bf16=True)
    assert res["wrong_blocks"] == 0 and res["worst_z"] < 1.0 and (res["z"] < z0).all()
