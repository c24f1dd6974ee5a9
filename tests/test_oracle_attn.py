"""The attention oracle (oracle/attn.py) against the reference's own outputs (tests/golden/attn.npz, written by
serve_attn.attn_check_torch / sample_python / recheck), and against what the mathematics fixes: a float64
softmax, one-key attention, a uniform key set, and scores of exact outputs."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import attn as OA
from tests._golden import as_f32, load, names, words

F = load("attn.npz")
NAMES = names(F)
COUNT_COLS = [OA.C_CALLS, OA.C_SAMPLES, OA.C_SKIP, OA.C_UNJ, OA.C_BADBLK, OA.C_KEYS, OA.C_WN, OA.C_WBAD,
              OA.C_WSLOT, OA.C_WLAST, OA.C_WWHERE]


def case(ci: int) -> dict:
    p = f"c{ci}_"
    dt = "fp16" if int(F[p + "dtype"]) else "bf16"
    ids = [str(s) for s in F[p + "ids"]]
    q, o, kv, key, val = (as_f32(words(F, n), dt) for n in ids)
    return {"q": q, "o": o, "kv": kv, "key": key, "val": val, "qsl": F[p + "qsl"], "seq_lens": F[p + "seq_lens"],
            "bt": F[p + "bt"], "slots": F[p + "slots"], "scale": float(F[p + "scale"]), "left": int(F[p + "left"]),
            "dtype": dt, "runs": F[p + "runs"]}


def zbits(key: int) -> float:
    return float(np.array([int(key) >> 32], np.uint32).view(np.float32)[0])


def run(c, step, nl, idx, active):
    return OA.check(c["q"], c["o"], c["kv"], c["key"], c["val"], c["qsl"], c["seq_lens"], c["bt"], c["slots"],
                    step=int(step), nl=int(nl), idx=int(idx), active=bool(active), scale=c["scale"],
                    left=c["left"], dtype=c["dtype"])


@pytest.mark.parametrize("ci", range(len(NAMES)), ids=NAMES)
def test_oracle_matches_the_reference_check(ci):
    c = case(ci)
    worst = 0.0
    for ri, (step, nl, idx, active) in enumerate(c["runs"]):
        p = f"c{ci}_r{ri}_"
        got = run(c, step, nl, idx, active)
        want = F[p + "state"]
        assert got.state[COUNT_COLS].tolist() == want[COUNT_COLS].tolist(), (ri, got.state, want)
        zr = F[p + "z"]
        for s in got.samples:
            if s.judged:
                fin = np.isfinite(zr[s.j])
                assert np.array_equal(np.isfinite(s.z), fin)
                d = np.abs(s.z[fin].astype(np.float64) - zr[s.j][fin])
                assert (d <= 1e-3 * np.maximum(1.0, zr[s.j][fin])).all(), (ri, s.j, d.max())
                worst = max(worst, float((d / np.maximum(1.0, zr[s.j][fin])).max(initial=0.0)))
        zw, zg = zbits(want[OA.C_ZT]), zbits(got.state[OA.C_ZT])
        assert zw == zg or abs(zw - zg) <= 1e-3 * max(1.0, zw)
        if zw > OA.ATTN_Z:                  # a located alarm: row, head, dim, step, position exactly
            for col in (OA.C_ZT, OA.C_ZH, OA.C_ZD, OA.C_ZS, OA.C_ZP):
                assert int(got.state[col]) & OA.M32 == int(want[col]) & OA.M32, (ri, col)
        cm = F[p + "capm"]
        assert got.capm[OA.CM_CLAIM] == cm[OA.CM_CLAIM]
        if cm[OA.CM_CLAIM]:
            keep = [k for k in range(OA.CAPM) if k != OA.CM_Z]
            assert got.capm[keep].tolist() == cm[keep].tolist()
            assert np.array_equal(got.capq, F[p + "capq"], equal_nan=True)
            assert np.array_equal(got.capo, F[p + "capo"], equal_nan=True)
    print(f"{NAMES[ci]}: max relative |dz| {worst:.2e}")


def test_sample_picks_match_sample_python():
    grid = F["pick_grid"]
    batches = {}
    for bi in range(int(grid[:, 0].max()) + 1):
        b = F[f"pick_b{bi}"].tolist()
        cut = b.index(-7)
        cut2 = b.index(-7, cut + 1)
        batches[bi] = (b[:cut], b[cut + 1:cut2], b[cut2 + 1], b[cut2 + 2])
    for bi, step, nl, idx, j, *want in grid.tolist():
        qsl, sls, rows, heads = batches[bi]
        s = OA.sample(step, idx, nl, j, qsl, sls, rows, heads)
        got = [-1] * 5 if s is None else [s["row"], s["request"], s["position"], s["seq_len"], s["head"]]
        assert got == want, (bi, step, nl, idx, j)


def test_recheck_matches_the_reference():
    for ri in range(4):
        q = as_f32(F[f"rc{ri}_q"], "bf16")
        kv = as_f32(F[f"rc{ri}_kv"], "bf16")
        D = q.shape[0]
        res = OA.recheck(q, F[f"rc{ri}_o"], kv[:, :D], kv[:, D:], float(F[f"rc{ri}_scale"]), "bf16")
        w = F[f"rc{ri}_res"]
        assert abs(res["worst_score"] - w[0]) <= 1e-9 * max(1.0, w[0])
        assert res["outputs_over_line"] == int(w[1]) and res["dim"] == int(w[2])
        assert (res["verdict"] == "output_wrong") == bool(w[5])


def test_the_check_checks_every_sample_kind_in_the_fixtures():
    """The fixtures exercise alarms, skipped samples, bad blocks, non-finite samples, wrong writes and slots."""
    tot = np.zeros(OA.COLS, np.int64)
    alarms = 0
    for ci in range(len(NAMES)):
        for ri in range(len(F[f"c{ci}_runs"])):
            st = F[f"c{ci}_r{ri}_state"]
            tot += np.where(np.arange(OA.COLS) >= OA.C_CALLS, st, 0)
            alarms += zbits(st[OA.C_ZT]) > OA.ATTN_Z
    for col in (OA.C_SAMPLES, OA.C_SKIP, OA.C_UNJ, OA.C_BADBLK, OA.C_WN, OA.C_WBAD, OA.C_WSLOT):
        assert tot[col] > 0, col
    assert alarms > 0


# -------------------------------------------------------------------------------- what the mathematics fixes
def _one_sample_case(L: int, D: int, seed: int, dtype="bf16"):
    """One decode request of L keys (one block-table row of 16-key blocks), one KV head, one query head."""
    rng = np.random.default_rng(seed)
    N = 16
    nb = -(-L // N)
    kv = rng.standard_normal((nb, 1, N, 2 * D)).astype(np.float32)
    kv = OA_round(kv, dtype)
    q = OA_round(rng.standard_normal((1, 1, D)).astype(np.float32) * 0.5, dtype)
    bt = np.arange(nb)[None, :]
    qsl = np.array([0, 1])
    sl = np.array([L])
    K = kv[:, 0, :, :D].reshape(-1, D)[:L].astype(np.float64)
    V = kv[:, 0, :, D:].reshape(-1, D)[:L].astype(np.float64)
    s = K @ q[0, 0].astype(np.float64) * D ** -0.5
    p = np.exp(s - s.max())
    o64 = (p / p.sum()) @ V
    return q, kv, bt, qsl, sl, o64


def OA_round(x, dtype):
    from oracle.lowp import round_to
    return round_to(x, dtype)


@pytest.mark.parametrize("L", [1, 17, 300])
def test_the_recompute_is_softmax_attention_and_a_rounded_output_scores_at_most_one(L):
    D = 64
    q, kv, bt, qsl, sl, o64 = _one_sample_case(L, D, L)
    o = OA_round(o64.astype(np.float32), "bf16").reshape(1, 1, D)
    out = OA.check(q, o, kv, np.zeros((1, 1, D)), np.zeros((1, 1, D)), qsl, sl, bt, np.array([-1]), step=0,
                   scale=D ** -0.5, has_write=False, samples=2)
    s0 = out.samples[0]
    assert s0.judged and s0.nkeys == L
    assert np.allclose(s0.ref, o64, rtol=2e-6, atol=1e-6)         # fp32 recompute = float64 softmax attention
    assert s0.zmax <= 1.0
    if L == 1:                                                     # one key: the output is its value exactly
        assert np.array_equal(s0.ref, kv[0, 0, 0, D:])


def test_a_uniform_key_set_averages_the_values():
    D, L = 64, 48
    q, kv, bt, qsl, sl, _ = _one_sample_case(L, D, 4)
    kv[:, :, :, :D] = kv[0, 0, 0, :D]                              # every key the same: p uniform
    out = OA.check(q, np.zeros((1, 1, D)), kv, np.zeros((1, 1, D)), np.zeros((1, 1, D)), qsl, sl, bt,
                   np.array([-1]), step=0, scale=D ** -0.5, has_write=False, samples=1)
    V = kv[:, 0, :, D:].reshape(-1, D)[:L].astype(np.float64)
    assert np.allclose(out.samples[0].ref, V.mean(0), rtol=1e-5, atol=1e-6)


def test_a_planted_mistake_in_the_oracle_is_caught_by_the_float64_softmax():
    """A dropped term (the max subtraction's rescale replaced by a wrong sign) must fail the float64 pin above."""
    D, L = 64, 40
    q, kv, bt, qsl, sl, o64 = _one_sample_case(L, D, 2)
    K = kv[:, 0, :, :D].reshape(-1, D)[:L].astype(np.float64)
    V = kv[:, 0, :, D:].reshape(-1, D)[:L].astype(np.float64)
    s = K @ q[0, 0].astype(np.float64) * D ** -0.5
    p_wrong = np.exp(-(s - s.max()))
    assert not np.allclose((p_wrong / p_wrong.sum()) @ V, o64, rtol=2e-6, atol=1e-6)


def test_bound_constants():
    u, sp, hp, g = OA.bound_consts("bf16", 128)
    assert (u, sp, hp, g) == (2 ** -8, 1e-37, 2 ** -126, 136 * 2 ** -23)
    u, sp, hp, g = OA.bound_consts("fp16", 64)
    assert (u, sp, hp, g) == (2 ** -11, 2 ** -24, 2 ** -25, 72 * 2 ** -23)
