"""The sampled fused-MoE recompute check (oracle: test infrastructure only; never imported by the library).

Restates serve_moe.py:106-258 in numpy: `sample_rows`, `recompute` (the routed experts' output with the fused
kernel's roundings, and the terms of its bound), `scores`, and one call of `moe_check_torch` (the state row's keys
and counts, the kept row, the routing-validity scan).  Matmuls are fp32 with numpy's summation order; the reference
and the HIP kernels each use their own, so recomputed values may differ by a rounding step where a sum crosses a
boundary (the bound's FLIPS term), and scores agree to a tolerance, counts and located faults exactly.
"""
from __future__ import annotations

import numpy as np

SAMPLES = 2
KAPPA, FLIPS, OUT_FLIPS = 1.0, 1.0, 2.0
M32 = 0xFFFFFFFF
ROW_A, ROW_B = 7919, 104729
ROWS_SHIFT, ROWS_MAX = 32, (1 << 31) - 1
C_ROW, C_COL, C_OUT, C_REF, C_STEP, C_CALLS, C_ROWS, C_UNJ, C_UNROUTED, C_PARTIAL, C_BADROW = range(11)
f32 = np.float32


def dtype_consts(dtype: str) -> tuple:
    if dtype == "fp16":
        return 2.0 ** -11, 2.0 ** -24, 65504.0
    return 2.0 ** -8, 1e-37, 3.3895313892515355e38


def rnd(v, dtype: str) -> np.ndarray:
    """float32 values rounded to bf16/fp16 (nearest, ties to even), as float32."""
    v = np.asarray(v, np.float32)
    if dtype == "fp16":
        with np.errstate(over="ignore"):
            return v.astype(np.float16).astype(np.float32)
    u = v.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(v), v, r).astype(np.float32)


def _erf(x):
    from math import erf
    return np.vectorize(lambda t: erf(float(t)), otypes=[np.float64])(x)


def act_fn(a, code: int):
    a = np.asarray(a, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        if code == 0:
            return (a / (f32(1.0) + np.exp(-a))).astype(np.float32)
        return (f32(0.5) * a * (f32(1.0) + _erf(a * f32(0.7071067811865476)).astype(np.float32))).astype(np.float32)


def dact_fn(a, code: int):
    a = np.asarray(a, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        if code == 0:
            s = (f32(1.0) / (f32(1.0) + np.exp(-a))).astype(np.float32)
            return (s * (f32(1.0) + a * (f32(1.0) - s))).astype(np.float32)
        cdf = (f32(0.5) * (f32(1.0) + _erf(a * f32(0.7071067811865476)).astype(np.float32))).astype(np.float32)
        return (cdf + a * np.exp(f32(-0.5) * a * a) * f32(0.3989422804014327)).astype(np.float32)


def sample_rows(step: int, rows: int, nlayers: int = 1) -> list:
    return [((step // max(nlayers, 1)) * ROW_A + j * ROW_B) % max(rows, 1) for j in range(SAMPLES)]


def recompute(x_rows, ids, g, w13, w2, expert_map, act: int, routed_first: bool, dtype: str) -> tuple:
    """serve_moe.py:127-169: (r, max_k |c_k|, sum_k g_k^2 sum_i (W2_ni h_i)^2, max_k,i |g_k W2_ni| s_i), [s, H]."""
    u = f32(dtype_consts(dtype)[0])
    x_rows = np.asarray(x_rows, np.float32)
    ids = np.asarray(ids, np.int64)
    g = np.asarray(g, np.float32)
    s, k = ids.shape
    H = w2.shape[1]
    r = np.zeros((s, H), np.float32)
    cmax = np.zeros((s, H), np.float32)
    sq = np.zeros((s, H), np.float32)
    mx = np.zeros((s, H), np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        for j in range(s):
            for kk in range(k):
                e = int(ids[j, kk])
                if expert_map is not None and e >= 0:
                    e = int(expert_map[e])
                if e < 0:
                    continue
                gk = g[j, kk]
                a = (np.asarray(w13[e], np.float32) @ x_rows[j]).astype(np.float32)
                if routed_first:
                    a = (a * gk).astype(np.float32)
                a = rnd(a, dtype)
                half = a.shape[0] // 2
                a1, a3 = a[:half], a[half:]
                s1 = rnd(act_fn(a1, act), dtype)
                h = rnd(s1 * a3, dtype)
                sens = (f32(2) * u * (np.abs(h) + np.abs(dact_fn(a1, act) * a1 * a3) + np.abs(s1 * a3))).astype(
                    np.float32)
                W = np.asarray(w2[e], np.float32)
                p = (W * h[None, :]).astype(np.float32)
                c = p.sum(1, dtype=np.float32)
                q = (p * p).sum(1, dtype=np.float32)
                m_ = (np.abs(W) * sens[None, :]).max(1).astype(np.float32)
                gw = f32(1.0) if routed_first else gk
                chat = rnd(c * gw, dtype)
                r[j] += chat
                cmax[j] = np.maximum(cmax[j], np.abs(chat))
                sq[j] += (q * gw * gw).astype(np.float32)
                mx[j] = np.maximum(mx[j], (m_ * abs(gw)).astype(np.float32))
    return r, cmax, sq, mx


def scores(y, r, cmax, sq, mx, dtype: str) -> tuple:
    """serve_moe.py:172-180: (z, judged)."""
    u, sp, fm = (f32(v) for v in dtype_consts(dtype))
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        den = (u * np.abs(r) + f32(OUT_FLIPS * 2) * u * cmax + f32(KAPPA) * u * np.sqrt(sq) + f32(FLIPS) * mx +
               sp).astype(np.float32)
        z = (np.abs(np.asarray(y, np.float32) - r) / den).astype(np.float32)
        judged = (np.abs(r) <= fm) & np.isfinite(den)
        z = np.where(judged, np.where(np.isnan(z), np.inf, z), f32(0))
    return z.astype(np.float32), judged


def _bits(v) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


def moe_check(x, out, topk_w, topk_ids, w13, w2, expert_map, act: int, routed_first: bool, dtype: str, state,
              cap: dict, raw: int, nlayers: int, index: int, line: float) -> tuple:
    """serve_moe.py:185-258 for one call: (state row after it, the kept row {meta, x, y, ids, g}, the sampled rows'
    scores [SAMPLES, H] (0 when not active))."""
    x = np.asarray(x, np.float32)
    out = np.asarray(out, np.float32)
    ids_all = np.asarray(topk_ids, np.int64)
    g_all = np.asarray(topk_w, np.float32)
    m, H = x.shape
    st = np.array(state, np.int64)
    cap = {k: np.array(v) for k, v in cap.items()}
    step = raw & M32
    active = step % max(nlayers, 1) == index
    real = (raw >> ROWS_SHIFT) & ROWS_MAX
    rows_n = min(real, m) if real > 0 else m
    rows = sample_rows(step, rows_n, nlayers)
    zs_out = np.zeros((SAMPLES, H), np.float32)
    if not active:
        return st, cap, zs_out
    xr, y = x[rows], out[rows]
    ids, g = ids_all[rows], g_all[rows]
    pad = (ids == -1).all(-1)
    r, cmax, sq, mx = recompute(xr, ids, g, w13, w2, expert_map, act, routed_first, dtype)
    z, judged = scores(y, r, cmax, sq, mx, dtype)
    judged = judged | pad[:, None]
    z = np.where(pad[:, None], f32(0), z)
    zs_out = z.copy()
    flat = z.reshape(-1)
    arg = int(np.argmax(flat))
    zmax = float(flat[arg])
    jrow, col = divmod(arg, H)
    row = rows[jrow]
    if zmax > 0:
        zb = _bits(zmax) << 32
        keys = [zb | row, zb | col, zb | _bits(y[jrow, col]), zb | _bits(r[jrow, col]), zb | step]
        st[:5] = np.maximum(st[:5], np.array(keys, np.int64))
    st[C_CALLS] += 1
    st[C_ROWS] += int((~pad).sum())
    st[C_UNJ] += int((~judged).sum())
    if real > 0:
        rr = min(real, m)
        nneg = (ids_all[:rr] == -1).sum(-1)
        k = ids_all.shape[1]
        none_ = nneg >= k
        some = (nneg > 0) & (nneg < k)
        st[C_UNROUTED] += int(none_.sum())
        st[C_PARTIAL] += int(some.sum())
        bad = np.nonzero(none_ | some)[0]
        if bad.size:
            st[C_BADROW] = max(int(st[C_BADROW]), (step << 32) | int(bad.max() + 1))
    if zmax > line and cap["meta"][0] == 0:
        cap["meta"] = np.array([1, row, step, _bits(zmax)], np.int64)
        cap["x"][:H] = xr[jrow]
        cap["y"][:H] = y[jrow]
        cap["ids"][:ids.shape[1]] = ids[jrow]
        cap["g"][:ids.shape[1]] = g[jrow]
    return st, cap, zs_out
