"""Oracle of the MoE router check (test infrastructure: only tests/ use it).

A numpy float32 restatement of the reference's serve_route.judge (serve_route.py:91-138) and of the state update of
route_check_torch (:141-186): for SAMPLES rows of a router call, were the chosen experts among the best the routing
policy allows (softmax or sigmoid scores, an optional correction bias for choosing, DeepSeek's grouped top-k) and
are the weights the chosen experts' scores, renormalized and scaled?  Tolerances as the reference's: ties within
TIE of a score's size (plus U_CHOICE unit roundoffs of 16-bit logits) may be picked either way, groups near the cut
within twice that; weights to W_ABS + (W_REL + U_WEIGHT u) |ref|.

Pinned by the reference's own answers on 165 seeded calls (tests/golden/route.npz: every policy, fp32 / bf16 /
fp16 logits, clean, moved and repeated experts, weights off and within the tolerance, ids out of range, padding,
ties, inactive steps) -- every row's verdicts and weight differences, the state row and the kept row.
"""
from __future__ import annotations

import numpy as np

SAMPLES = 2
TIE = 1e-6
W_ABS, W_REL = 2e-5, 1e-4
U_CHOICE, U_WEIGHT = 4.0, 6.0
ROW_A, ROW_B = 7919, 104729
M32 = 0xFFFFFFFF
S31 = 0x7FFFFFFF
COLS = 6
C_CALLS, C_SET, C_WEIGHT, C_LAST, C_WDIFF, C_ROWS = range(COLS)
KIND_SET, KIND_WEIGHT = 2, 1
F32 = np.float32


def unit_roundoff(dtype: str) -> float:
    """Half the epsilon of 16-bit logits; 0 for fp32 (serve_route.py:68-70)."""
    return {"bf16": 2.0 ** -8, "fp16": 2.0 ** -11}.get(dtype, 0.0)


def _tol(v: np.ndarray, u: float) -> np.ndarray:
    """serve_route.py:73-75: TIE of the size (at least 1) plus U_CHOICE unit roundoffs; an infinite size counts 0."""
    a = np.abs(v).astype(F32)
    a = np.where(np.isinf(a), F32(0), a)
    return (F32(TIE) * np.maximum(a, F32(1)) + F32(U_CHOICE * u) * a).astype(F32)


def _scores(lf: np.ndarray, scoring: int) -> np.ndarray:
    if scoring == 0:
        e = np.exp(lf - lf.max(-1, keepdims=True))
        return (e / e.sum(-1, keepdims=True)).astype(F32)
    return (F32(1) / (F32(1) + np.exp(-lf))).astype(F32)


def _kth_largest(v: np.ndarray, k: int) -> np.ndarray:
    """k-th largest along the last axis, counting equal values each (torch.topk(k).values[..., -1])."""
    return -np.sort(-v, axis=-1)[..., k - 1]


def _group_scores(g: np.ndarray, biased: bool) -> np.ndarray:
    """A group's score (serve_route.py:106): its two best choice scores summed with a correction bias, else its
    best one."""
    if biased:
        top2 = -np.sort(-g, axis=-1)[..., :2]
        return (top2[..., 0] + top2[..., 1]).astype(F32)
    return g.max(-1)


def judge(lf, kid, kw, k, scoring, renormalize, bias, groups, topk_group, scale, u):
    """Rows of fp32 logits lf [r, E] against the router's ids and weights [r, k] (serve_route.py:91-138):
    (wrong expert set [r], wrong weight [r], weight differences [r, k])."""
    lf = np.asarray(lf, F32)
    kid = np.asarray(kid, np.int64)
    kw = np.asarray(kw, F32)
    r, e = lf.shape
    s = _scores(lf, scoring)
    choice = (s + np.asarray(bias, F32)[None, :]).astype(F32) if bias is not None else s
    valid = (kid >= 0) & (kid < e)
    kc = np.clip(kid, 0, e - 1)
    thr = np.ones_like(choice, dtype=bool)
    allow = np.ones_like(choice, dtype=bool)
    if groups:
        gsz = e // groups
        g = choice.reshape(r, groups, gsz)
        gs = _group_scores(g, bias is not None)
        srt = -np.sort(-gs, axis=-1)
        gth = srt[:, topk_group - 1]
        gnext = srt[:, topk_group] if topk_group < groups else np.full_like(gth, -np.inf)
        tolg = (F32(2) * _tol(gth, u))[:, None]
        amb = gnext[:, None] >= (gth[:, None] - tolg)
        clear = gs >= gth[:, None]
        thr_g = np.where(amb, gs > gth[:, None] + tolg, clear)
        allow_g = np.where(amb, gs >= gth[:, None] - tolg, clear)
        thr = np.repeat(thr_g, gsz, axis=1)
        allow = np.repeat(allow_g, gsz, axis=1)
    bound = np.repeat(_kth_largest(np.where(thr, choice, -np.inf).astype(F32), k)[:, None], k, axis=1)
    if groups:
        kwg = _kth_largest(g, k) if gsz >= k else np.full_like(gs, -np.inf)
        low = np.sort(np.where(allow_g, kwg, np.inf), axis=-1)[:, topk_group - 1]
        bound = np.maximum(np.maximum(bound, low[:, None]), np.take_along_axis(kwg, kc // gsz, 1))
    ck = np.take_along_axis(choice, kc, 1)
    ok = valid & np.take_along_axis(allow, kc, 1) & (ck >= (bound - _tol(bound, u)))
    srt_id = np.sort(kid, axis=-1)
    dup = (srt_id[:, 1:] == srt_id[:, :-1]).any(-1) if k > 1 else np.zeros(r, bool)
    set_bad = ~ok.all(-1) | dup
    sk = np.where(valid, np.take_along_axis(s, kc, 1), F32(0)).astype(F32)
    ref = (sk / (sk.sum(-1, keepdims=True) + F32(1e-20))).astype(F32) if renormalize else sk
    ref = (ref * F32(scale)).astype(F32)
    diff = np.where(valid, np.abs(kw - ref), F32(0)).astype(F32)
    lim = (F32(W_ABS) + F32(W_REL + U_WEIGHT * u) * np.abs(ref)).astype(F32)
    w_bad = (~(diff <= lim)).any(-1) & ~set_bad
    return set_bad, w_bad, diff


def sample_rows(step: int, real: int, nlayers: int) -> np.ndarray:
    """serve_route.py:78-82."""
    return np.array([((step // max(nlayers, 1)) * ROW_A + j * ROW_B) % max(real, 1) for j in range(SAMPLES)],
                    np.int64)


def route_check(logits, w, ids, k, scoring, renormalize, bias, groups, topk_group, scale, dtype, real, step,
                nlayers, index, state=None, cap=None):
    """One call of serve_route.route_check_torch (serve_route.py:141-184) on fp32 logits (the 16-bit ones already
    widened; `dtype` names what they were): returns (state [COLS] int64, kept (meta [6], logits, ids, weights) or
    None).  The kept row is the first sampled row found wrong."""
    logits = np.asarray(logits, F32)
    m, e = logits.shape
    state = np.zeros(COLS, np.int64) if state is None else state.copy()
    real = min(max(int(real), 0), m)
    step = int(step) & M32
    live = real > 0 and step % max(nlayers, 1) == index
    rows = sample_rows(step, real, nlayers)
    u = unit_roundoff(dtype)
    lf, kid, kw = logits[rows], np.asarray(ids, np.int64)[rows], np.asarray(w, F32)[rows]
    sb, wb, diff = judge(lf, kid, kw, k, scoring, renormalize, bias, groups, topk_group, scale, u)
    judged = live & ~(kid == -1).all(-1)
    sb, wb = sb & judged, wb & judged
    state[C_CALLS] += int(live)
    state[C_ROWS] += int(judged.sum())
    state[C_SET] += int(sb.sum())
    state[C_WEIGHT] += int(wb.sum())
    kind = np.where(sb, KIND_SET, np.where(wb, KIND_WEIGHT, 0))
    rec = np.where(kind > 0, ((step & S31) << 32) | (kind << 24) | (rows & 0xFFFFFF), 0)
    state[C_LAST] = max(int(state[C_LAST]), int(rec.max()))
    worst = F32(np.where(judged[:, None], diff, F32(0)).max())
    state[C_WDIFF] = max(int(state[C_WDIFF]), int(np.array([worst], F32).view(np.uint32)[0]))
    bad = sb | wb
    kept = None
    if bad.any() and (cap is None or cap == 0):
        jb = int(np.argmax(bad))
        code = {"fp32": 0, "bf16": 1, "fp16": 2}[dtype]
        kept = (np.array([1, rows[jb], step, kind[jb], e, code], np.int64), lf[jb].copy(), kid[jb].copy(),
                kw[jb].copy())
    return state, kept


def bad_rows(logits, w, ids, k, scoring, renormalize, bias, groups, topk_group, scale, dtype, real, step,
             nlayers) -> list:
    """The sampled rows a call finds wrong (the rows a GPU may keep: its samples race to be the kept one)."""
    rows = sample_rows(int(step) & M32, min(max(int(real), 0), np.asarray(logits).shape[0]), nlayers)
    lf, kid = np.asarray(logits, F32)[rows], np.asarray(ids, np.int64)[rows]
    sb, wb, _ = judge(lf, kid, np.asarray(w, F32)[rows], k, scoring, renormalize, bias, groups, topk_group, scale,
                      unit_roundoff(dtype))
    judged = ~(kid == -1).all(-1)
    return [int(r) for r, b in zip(rows, (sb | wb) & judged) if b]
