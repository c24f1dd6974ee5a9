"""The fingerprint oracle pinned by published values and brute force (no fixture needed: closed forms).

  * splitmix64: the mix of position + golden gamma at p = 0 is splitmix64's first output from state 0,
    0xE220A8397B1DCDAF, and the mix of 2 * gamma its second, 0x6E789E6AA1B965F4 (Steele, Lea, Flood 2014;
    the values every splitmix64 implementation publishes);
  * numpy (uint64 wrapping) == Python ints (exact, mod 2^64) == the C file, on random words and extremes;
  * the reference's own formulation with signed int64 and masked arithmetic shifts (recompute.py:93-106,
    serve_weights.py:164-169), restated in numpy int64, gives the same weights and keys;
  * the reference tests' known patterns (test_recompute.py:169-334, test_serve_weights.py:181-213).
"""
from __future__ import annotations

import numpy as np

from oracle import fingerprint as F


def _mix(z):
    z &= F.MASK
    z = ((z ^ (z >> 30)) * F.FP_M1) & F.MASK
    z = ((z ^ (z >> 27)) * F.FP_M2) & F.MASK
    return z ^ (z >> 31)


def test_splitmix64_published_outputs():
    assert _mix(F.FP_SEED) == 0xE220A8397B1DCDAF
    assert _mix(2 * F.FP_SEED) == 0x6E789E6AA1B965F4
    assert _mix(3 * F.FP_SEED) == 0x06C45D188009454F
    w1, _ = F.fp3_weights_py(0)
    assert w1 == 0xE220A8397B1DCDAF | 1


def _lsr(z, s):
    return (z >> s) & ((1 << (64 - s)) - 1)


def test_fp3_weights_match_the_signed_int64_formulation():
    pos = np.arange(0, 200_000, 7, dtype=np.int64)
    with np.errstate(over="ignore"):
        z = pos + np.int64(-7046029254386353131)
        z = (z ^ _lsr(z, 30)) * np.int64(-4658895280553007687)
        z = (z ^ _lsr(z, 27)) * np.int64(-7723592293110705685)
        z = z ^ _lsr(z, 31)
        w1s, w2s = z | 1, (z ^ _lsr(z, 32)) | 1
    w1, w2 = F.fp3_weights(pos.astype(np.uint64))
    assert np.array_equal(w1.view(np.int64), w1s) and np.array_equal(w2.view(np.int64), w2s)


def test_fp2_keys_match_the_signed_int64_formulation():
    low31 = (1 << 31) - 1
    pos = np.arange(0, 100_000, 3, dtype=np.int64)
    with np.errstate(over="ignore"):
        h = pos ^ np.int64(0x2545F4914F6CDD1D)
        h = (h ^ ((h >> 33) & low31)) * np.int64(0xFF51AFD7ED558CCD - (1 << 64))
        h = (h ^ ((h >> 33) & low31)) * np.int64(0xC4CEB9FE1A85EC53 - (1 << 64))
        h = h ^ ((h >> 33) & low31)
    assert np.array_equal(F.fp2_keys(pos.astype(np.uint64)).view(np.int64), h)


def test_fp3_three_ways_agree():
    rng = np.random.default_rng(1)
    for n in (1, 9, 1000, 4097):
        w = rng.integers(-32768, 32768, n).astype(np.int16)
        w[:2] = [-32768, 32767][:n]
        assert tuple(F.fp3(w)) == F.fp3_py(w)
        if F.c_lib() is not None:
            assert np.array_equal(F.fp3_c(w), F.fp3(w))
        w8 = rng.integers(-128, 128, n).astype(np.int8)
        assert tuple(F.fp3(w8)) == F.fp3_py(w8)
    big = rng.integers(-32768, 32768, 3_000_000).astype(np.int16)
    if F.c_lib() is not None:
        assert np.array_equal(F.fp3_c(big), F.fp3(big))


def test_fp2_matches_the_reference_tests_python_reference():
    """test_serve_weights.py:181-213: values as signed (16, 32 bits) or unsigned (8 bits) integers, extremes."""
    rng = np.random.default_rng(4)
    for dt, bits in ((np.int16, 16), (np.int32, 32), (np.uint8, 8)):
        if bits > 8:
            w = rng.integers(-(1 << (bits - 1)), 1 << (bits - 1), 97).astype(dt)
            w[0], w[1] = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
        else:
            w = rng.integers(0, 256, 97).astype(dt)
            w[0], w[1] = 0, 255
        assert tuple(F.fp2(w)) == F.fp2_py(w)
    d = rng.standard_normal(33)
    assert tuple(F.fp2(F.fp2_words(d))) == F.fp2_py(d.view(np.int32))


def test_fp3_sees_the_reference_tests_patterns():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(1000).astype(np.float32)
    xw = F.fp3_words(x).copy()
    f = F.fp3(xw)
    for i in (0, 251, 252, 1999):
        y = xw.copy()
        y[i] ^= 1
        assert not np.array_equal(F.fp3(y), f)
    y = xw.copy()
    y[10] += 1
    y[11] -= 2
    y[12] += 1
    assert not np.array_equal(F.fp3(y), f)
    z = np.zeros(1000, np.float32)
    z.view(np.uint32)[3] = 0x3F800000
    z.view(np.uint32)[600] = 0x3F7F0001
    s = z.copy()
    s[3], s[600] = z[600], z[3]
    assert not np.array_equal(F.fp3(F.fp3_words(z)), F.fp3(F.fp3_words(s)))
    w1, w2 = F.fp3_weights(np.arange(100_000, dtype=np.uint64))
    assert bool((w1 & 1).all()) and bool((w2 & 1).all())
    assert np.unique(w1).size == np.unique(w2).size == 100_000


def test_kv_block_fp3_is_the_per_block_fingerprint():
    rng = np.random.default_rng(2)
    cache = rng.integers(-32768, 32768, (6, 8, 16, 32)).astype(np.int16)
    out = F.kv_block_fp3(cache)
    for b in range(6):
        assert np.array_equal(out[b], F.fp3(cache[b].reshape(-1)))
    if F.c_lib() is not None:
        assert np.array_equal(F.kv_block_fp3_c(cache, threads=3), out)
