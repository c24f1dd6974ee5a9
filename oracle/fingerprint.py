"""Integer fingerprints of raw tensor bits (oracle: test infrastructure only).

Two families, both sums of words times position weights, mod 2^64 (wrapping, so order-independent):

fp3 -- recompute.py:59-61 (constants), :93-116 (`_lsr`, `_fp_weights`, `_fingerprint_torch`), _fingerprint.py:51-65
    words b = the tensor's 16-bit words as signed int16 (8-bit words as signed int8 for 1-byte dtypes),
    position p = word index; z = p + SEED; z = (z ^ z>>>30) * M1; z = (z ^ z>>>27) * M2; z ^= z>>>31;
    w1 = z | 1; w2 = (z ^ z>>>32) | 1;   result (sum b, sum b*w1, sum b*w2) as int64.
    (z is splitmix64's output mixing applied to p + golden gamma: z(0) is splitmix64's first output from state
    0, 0xE220A8397B1DCDAF, and the mix of 2 * gamma its second, 0x6E789E6AA1B965F4 -- published values the
    tests pin it with.)

fp2 -- serve_weights.py:73-86 (constants), :151-185 (`_int_view`, `keys`, `fingerprint`)
    words x = int16 for 2-byte dtypes, int32 for 4-byte, int32 halves for 8-byte, uint8 for 1-byte;
    key k(i) = fmix64(i ^ KEY_SEED) (MurmurHash3's 64-bit finalizer);  result (sum x, sum x*k(i)) as int64.

Both are given here three ways: numpy uint64 arrays (vectorized), Python ints (brute force, tiny inputs),
and the C file fingerprint.c (fast, for the CPU baseline), which tests check against each other.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

MASK = (1 << 64) - 1
FP_SEED = 0x9E3779B97F4A7C15           # recompute.py:59 (-7046029254386353131 as int64)
FP_M1 = 0xBF58476D1CE4E5B9             # recompute.py:60
FP_M2 = 0x94D049BB133111EB             # recompute.py:61
KEY_SEED = 0x2545F4914F6CDD1D          # serve_weights.py:75
MIX1 = 0xFF51AFD7ED558CCD              # serve_weights.py:76
MIX2 = 0xC4CEB9FE1A85EC53              # serve_weights.py:77

_U = np.uint64


def _s64(v: int) -> int:
    v &= MASK
    return v - (1 << 64) if v >> 63 else v


# ---------------------------------------------------------------- fp3 (recompute)
def fp3_weights_py(p: int):
    z = (p + FP_SEED) & MASK
    z = ((z ^ (z >> 30)) * FP_M1) & MASK
    z = ((z ^ (z >> 27)) * FP_M2) & MASK
    z = z ^ (z >> 31)
    return z | 1, (z ^ (z >> 32)) | 1


def fp3_py(words) -> tuple:
    """Brute force with Python ints: words are signed integers (int16 or int8 values)."""
    s0 = s1 = s2 = 0
    for p, b in enumerate(int(w) for w in words):
        w1, w2 = fp3_weights_py(p)
        s0 += b
        s1 += b * w1
        s2 += b * w2
    return tuple(_s64(v) for v in (s0, s1, s2))


def fp3_weights(pos: np.ndarray):
    z = pos.astype(_U) + _U(FP_SEED)
    z = (z ^ (z >> _U(30))) * _U(FP_M1)
    z = (z ^ (z >> _U(27))) * _U(FP_M2)
    z = z ^ (z >> _U(31))
    return z | _U(1), (z ^ (z >> _U(32))) | _U(1)


def fp3_words(t: np.ndarray) -> np.ndarray:
    """The words fp3 sums: int16 view (or int8 for 1-byte elements) of a contiguous array; recompute.py:86-87."""
    a = np.ascontiguousarray(t).reshape(-1)
    return a.view(np.int16) if a.dtype.itemsize % 2 == 0 else a.view(np.int8)


def fp3(words: np.ndarray, start: int = 0, chunk: int = 1 << 22) -> np.ndarray:
    """(3,) int64 of signed words (int16 / int8 array); positions start at `start`."""
    words = np.asarray(words).reshape(-1)
    out = np.zeros(3, _U)
    for i in range(0, words.size, chunk):
        b = words[i:i + chunk].astype(np.int64).astype(_U)
        w1, w2 = fp3_weights(np.arange(start + i, start + i + b.size, dtype=np.uint64))
        out += np.array([b.sum(dtype=_U), (b * w1).sum(dtype=_U), (b * w2).sum(dtype=_U)], _U)
    return out.view(np.int64)


# ---------------------------------------------------------------- fp2 (serve_weights)
def fmix64_py(h: int) -> int:
    h &= MASK
    h = ((h ^ (h >> 33)) * MIX1) & MASK
    h = ((h ^ (h >> 33)) * MIX2) & MASK
    return h ^ (h >> 33)


def fp2_py(words) -> tuple:
    s0 = s1 = 0
    for i, x in enumerate(int(w) for w in words):
        s0 += x
        s1 += x * fmix64_py(i ^ KEY_SEED)
    return _s64(s0), _s64(s1)


def fp2_keys(pos: np.ndarray) -> np.ndarray:
    h = pos.astype(_U) ^ _U(KEY_SEED)
    h = (h ^ (h >> _U(33))) * _U(MIX1)
    h = (h ^ (h >> _U(33))) * _U(MIX2)
    return h ^ (h >> _U(33))


def fp2_words(t: np.ndarray) -> np.ndarray:
    """serve_weights.py:151-161: int16 for 2-byte elements, int32 for 4 and 8 (halves), uint8 for 1."""
    a = np.ascontiguousarray(t).reshape(-1)
    es = a.dtype.itemsize
    if es == 2:
        return a.view(np.int16)
    if es in (4, 8):
        return a.view(np.int32)
    return a.view(np.uint8)


def fp2(words: np.ndarray, start: int = 0, chunk: int = 1 << 22) -> np.ndarray:
    words = np.asarray(words).reshape(-1)
    out = np.zeros(2, _U)
    for i in range(0, words.size, chunk):
        x = words[i:i + chunk].astype(np.int64).astype(_U)
        k = fp2_keys(np.arange(start + i, start + i + x.size, dtype=np.uint64))
        out += np.array([x.sum(dtype=_U), (x * k).sum(dtype=_U)], _U)
    return out.view(np.int64)


# ---------------------------------------------------------------- paged-KV block fingerprints
def kv_block_fp3(cache: np.ndarray) -> np.ndarray:
    """(blocks, 3) int64: fp3 of every block of a paged cache (blocks on axis 0), each block's words numbered
    from 0 -- the fingerprint recompute.fingerprint gives the block as a tensor of its own."""
    nblk = cache.shape[0]
    words = fp3_words(cache).reshape(nblk, -1)
    w = words.astype(np.int64).astype(_U)
    w1, w2 = fp3_weights(np.arange(words.shape[1], dtype=np.uint64))
    out = np.stack([w.sum(1, dtype=_U), (w * w1).sum(1, dtype=_U), (w * w2).sum(1, dtype=_U)], axis=1)
    return out.view(np.int64)


# ---------------------------------------------------------------- the C version
_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = [None]


def c_lib():
    """oracle/_build/liboracle_fp.so (built by oracle/Makefile), or None."""
    if _LIB[0] is None:
        path = os.path.join(_HERE, "_build", "liboracle_fp.so")
        if not os.path.exists(path):
            return None
        lib = ctypes.CDLL(path)
        for name in ("oracle_fp3_i16", "oracle_fp3_i8", "oracle_kv_fp3_i16"):
            getattr(lib, name).restype = None
        lib.oracle_fp3_i16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_fp3_i8.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_kv_fp3_i16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                          ctypes.c_int]
        _LIB[0] = lib
    return _LIB[0]


def fp3_c(words: np.ndarray) -> np.ndarray:
    lib = c_lib()
    words = np.ascontiguousarray(words).reshape(-1)
    out = np.zeros(3, np.int64)
    fn = lib.oracle_fp3_i16 if words.dtype.itemsize == 2 else lib.oracle_fp3_i8
    fn(words.ctypes.data, words.size, 0, out.ctypes.data)
    return out


def kv_block_fp3_c(cache: np.ndarray, threads: int = 1) -> np.ndarray:
    lib = c_lib()
    a = np.ascontiguousarray(cache)
    nblk = a.shape[0]
    words = a.reshape(-1).view(np.int16)
    out = np.zeros((nblk, 3), np.int64)
    lib.oracle_kv_fp3_i16(words.ctypes.data, nblk, words.size // max(1, nblk), out.ctypes.data, int(threads))
    return out
