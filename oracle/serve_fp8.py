"""The FP8 quantization check (oracle: test infrastructure only; never imported by the library).

Restates serve_fp8.py:63-178 in numpy: `quant_check_torch` for one call, from the layer input x2 (float32 values of
its bf16/fp16/fp32 elements), the FP8 codes the GEMM got, their scale(s) and the step's real rows, returning the
layer's 8-column state row after the call.  The E4M3 ("fn": no infinities, S.1111.111 NaN) conversion is written
out from the format (round to nearest even, NaN keeps its sign) and pinned against torch's float8_e4m3fn conversion
in tests/test_oracle_fp8.py.
"""
from __future__ import annotations

import numpy as np

FP8_MAX = np.float32(448.0)
MIN_SCALE = np.float32(1.0 / (448.0 * 512.0))
SAMPLES = 2
SCALE_TOL = np.float32(2.0 ** -8)
TINY = np.float32(1e-38)
ROW_A, ROW_B = 7919, 104729
M32, S31, EVERY_ROW = 0xFFFFFFFF, 0x7FFFFFFF, 0xFFFFFF
C_CALLS, C_SCALE, C_OUTSIDE, C_VALUES, C_ONE, C_LAST, C_RATIO, C_STATIC = range(8)
KIND_SCALE, KIND_OUTSIDE, KIND_VALUES, KIND_STATIC = 1, 2, 3, 4


def to_e4m3(v) -> np.ndarray:
    """float32 values (|v| <= 448 or NaN) -> E4M3 codes (uint8), round to nearest even."""
    v = np.asarray(v, np.float32)
    u = v.view(np.uint32).astype(np.int64)
    sign = (u >> 24) & 0x80
    a = u & 0x7FFFFFFF
    out = np.zeros(v.shape, np.int64)
    nan = a > 0x7F800000
    sub = (a < 0x3C800000) & ~nan                     # |v| < 2^-6: multiples of 2^-9
    with np.errstate(invalid="ignore"):
        f = np.abs(v).astype(np.float64) * 512.0      # exact
        fl = np.floor(f)
        frac = f - fl
        rne = np.where(frac > 0.5, fl + 1, np.where(frac < 0.5, fl, fl + (fl % 2)))
    rne = np.where(sub, rne, 0.0)
    out[sub] = rne[sub].astype(np.int64)
    nor = ~sub & ~nan
    r = (a + 0x7FFFF + ((a >> 20) & 1)) >> 20         # exponent and 3 mantissa bits, rounded to nearest even
    out[nor] = r[nor] - (120 << 3)
    out[nan] = 0x7F
    return (out | sign).astype(np.uint8)


def fp8_order(codes) -> np.ndarray:
    c = np.asarray(codes).astype(np.int64)
    mag = c & 0x7F
    return np.where(c & 0x80, -mag, mag)


def _amax(x) -> np.float32:
    """max |x| as torch's amax: NaN if any element is NaN, 0 over nothing."""
    x = np.abs(np.asarray(x, np.float32))
    if x.size == 0:
        return np.float32(0.0)
    return np.float32(np.max(x))


def _quantize(row, scale: np.float32, divide: bool) -> np.ndarray:
    xf = np.asarray(row, np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        v = (xf / scale) if divide else (xf * (np.float32(1.0) / scale))
        v = np.where(np.isnan(v), v, np.clip(v, -FP8_MAX, FP8_MAX)).astype(np.float32)
    return to_e4m3(v)


def quant_check(x2, xq, xs, recipe: int, scale_ub, static_ref, real_rows: int, step: int, mult: int = 1,
                state=None) -> np.ndarray:
    """serve_fp8.py:79-178.  x2 (m, k) float32 values; xq (m' >= m, k) uint8 codes; xs float32 scale(s) (per token:
    one per row of xq); recipe 0 static, 1 per tensor, 2 per token; real_rows: the device's rows count (before
    mult); returns the state row (8 int64) after adding this call to `state`."""
    x2 = np.asarray(x2, np.float32)
    xq = np.asarray(xq, np.uint8)
    xs = np.asarray(xs, np.float32).reshape(-1)
    m = x2.shape[0]
    st = np.zeros(8, np.int64) if state is None else np.array(state, np.int64)
    real = min(max(int(real_rows) * int(mult), 0), m)
    armed = real > 0
    step = int(step) & M32
    rows = [(step * ROW_A + j * ROW_B) % max(real, 1) for j in range(SAMPLES)]
    mult = max(int(mult), 1)
    scale_bad, outside, static_bad = False, False, False
    ratio = np.float32(1.0)
    scale_row = EVERY_ROW
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        if recipe == 1:
            ks = xs[0]
            ref = np.float32(_amax(x2[:real]) / FP8_MAX)
            every = np.float32(_amax(x2) / FP8_MAX)
            scale_bad = bool(abs(ks - ref) > SCALE_TOL * abs(ref) + TINY)
            outside = scale_bad and bool(abs(ks - every) <= SCALE_TOL * abs(every) + TINY) and bool(every > ref)
            ratio = np.float32(ks / (ref if np.isnan(ref) else max(ref, TINY)))
            use = [ks] * SAMPLES
            divide = False
        elif recipe == 2:
            use, diffs, ratios = [], [], []
            for r in rows:
                amax = _amax(x2[r])
                if scale_ub is not None:
                    ub = np.float32(np.asarray(scale_ub, np.float32).reshape(-1)[0])
                    amax = np.float32(np.nan) if (np.isnan(amax) or np.isnan(ub)) else min(amax, ub)
                ref = np.float32(amax / FP8_MAX)
                ref = ref if np.isnan(ref) else max(ref, MIN_SCALE)
                ks = xs[min(r, xs.size - 1)]
                use.append(ks)
                diffs.append(bool(abs(ks - ref) > SCALE_TOL * abs(ref) + TINY))
                ratios.append(np.float32(ks / (ref if np.isnan(ref) else max(ref, TINY))))
            sel = diffs.index(True) if any(diffs) else 0
            scale_bad = any(diffs)
            ratio = ratios[sel]
            scale_row = rows[sel] // mult
            divide = True
        else:
            use = [xs[0]] * SAMPLES
            divide = False
            if static_ref is not None:
                static_bad = not bool(xs[0] == np.float32(np.asarray(static_ref, np.float32).reshape(-1)[0]))
    nbad, n_one = [], 0
    for j, r in enumerate(rows):
        d = np.abs(fp8_order(_quantize(x2[r], np.float32(use[j]), divide)) - fp8_order(xq[r]))
        nbad.append(int((d >= 2).sum()))
        n_one += int((d == 1).sum())
    vb = [nb > 0 and armed for nb in nbad]
    sb = scale_bad and armed
    if armed:
        st[C_CALLS] += 1
        st[C_SCALE] += int(sb)
        st[C_OUTSIDE] += int(outside)
        st[C_VALUES] += sum(vb)
        st[C_ONE] += n_one
        st[C_STATIC] = max(st[C_STATIC], int(static_bad))
    kind = KIND_OUTSIDE if (outside and armed) else KIND_SCALE if sb else KIND_VALUES if any(vb) else \
        KIND_STATIC if (static_bad and armed) else 0
    val_row = rows[vb.index(True) if any(vb) else 0] // mult
    bad_row = val_row if kind == KIND_VALUES else scale_row if kind == KIND_SCALE else EVERY_ROW
    rec = ((step & S31) << 32) | (kind << 24) | (bad_row & 0xFFFFFF)
    if kind > 0:
        st[C_LAST] = max(st[C_LAST], rec)
    if sb:
        r_ = np.float32(abs(ratio))
        r_ = r_ if np.isnan(r_) else np.float32(min(r_, np.float32(3e38)))
        st[C_RATIO] = max(st[C_RATIO], int(np.array([r_], np.float32).view(np.uint32)[0]))
    return st
