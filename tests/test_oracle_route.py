"""The MoE router check's oracle (oracle/route.py) against the reference's answers (tests/golden/route.npz:
serve_route.judge on every row of 165 seeded router calls, and route_check_torch's state row and kept row).

Every row's wrong-set and wrong-weight verdicts, the state row's counts and packed last finding, and the kept row
exactly; weight differences to 1e-6 of the weights' size plus 3e-7 (a few float32 ulps of weights up to 2.5: exp and
sums from another library, in another order); the worst weight difference the state keeps to the same.  Planted
mistakes in the oracle (the correction bias dropped from the choice, a biased group scored by its best expert alone,
the renormalization skipped) each fail."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import route as R
from tests import _golden as G

RT = G.load("route.npz")
NAMES = G.names(RT)
DT = {0: "fp32", 1: "bf16", 2: "fp16"}


def route_case(i: int) -> dict:
    p = f"c{i}_"
    E, k, scoring, renorm, groups, tg, code, step, real, nl, idx = (int(v) for v in RT[p + "meta"])
    dt = DT[code]
    if dt == "fp32":
        logits = RT[p + "logits"].astype(np.float32)
        bits = None
    else:
        bits = RT[p + "logits_bits"]
        logits = G.as_f32(bits, dt).reshape(bits.shape)
    bias = RT[p + "bias"]
    return dict(name=NAMES[i], E=E, k=k, scoring=scoring, renorm=bool(renorm), groups=groups, tg=tg, dt=dt,
                step=step, real=real, nl=nl, idx=idx, logits=logits, bits=bits, ids=RT[p + "ids"],
                w=RT[p + "w"], bias=bias if bias.size else None, scale=float(RT[p + "scale"]),
                state=RT[p + "state"], cap_meta=RT[p + "cap_meta"], cap_lg=RT[p + "cap_lg"],
                cap_ids=RT[p + "cap_ids"], cap_w=RT[p + "cap_w"], set_bad=RT[p + "set_bad"], w_bad=RT[p + "w_bad"],
                diff=RT[p + "diff"])


def _f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", int(bits) & 0xFFFFFFFF))[0]


def state_agrees(got, want) -> list:
    """Columns of a state row that differ (the worst weight difference to 1e-6 relative + 3e-7)."""
    bad = []
    for c in range(R.COLS):
        if c == R.C_WDIFF:
            a, b = _f32(got[c]), _f32(want[c])
            if abs(a - b) > 1e-6 * abs(b) + 3e-7:
                bad.append((c, a, b))
        elif int(got[c]) != int(want[c]):
            bad.append((c, int(got[c]), int(want[c])))
    return bad


def run_oracle(c: dict, **over):
    return R.route_check(c["logits"], c["w"], c["ids"], c["k"], c["scoring"], c["renorm"], c["bias"], c["groups"],
                         c["tg"], c["scale"], c["dt"], c["real"], c["step"], c["nl"], c["idx"])


def test_fixture_inventory():
    assert len(NAMES) == 165
    for pol in ("softmax_top4", "sigmoid_top6", "biased_top4", "deepseek_grouped", "grouped_softmax",
                "grouped_small_groups"):
        for case in ("clean", "moved_expert", "repeated_expert", "weights_off", "id_out_of_range", "padding"):
            assert any(n.startswith(pol) and n.endswith(case) for n in NAMES), (pol, case)


@pytest.mark.parametrize("i", range(len(NAMES)))
def test_every_row_judged_as_the_reference_judges_it(i):
    c = route_case(i)
    sb, wb, diff = R.judge(c["logits"], c["ids"], c["w"], c["k"], c["scoring"], c["renorm"], c["bias"],
                           c["groups"], c["tg"], c["scale"], R.unit_roundoff(c["dt"]))
    assert np.array_equal(sb, c["set_bad"]) and np.array_equal(wb, c["w_bad"]), (c["name"], sb, wb)
    tol = 1e-6 * np.abs(c["w"]) + 3e-7                   # (a few ulps of the weights: exp in another library)
    assert (np.abs(diff - c["diff"]) <= tol).all(), (c["name"], np.abs(diff - c["diff"]).max())


@pytest.mark.parametrize("i", range(len(NAMES)))
def test_state_and_kept_row_match_reference(i):
    c = route_case(i)
    st, kept = run_oracle(c)
    assert not state_agrees(st, c["state"]), (c["name"], state_agrees(st, c["state"]))
    if kept is None:
        assert not c["cap_meta"].any(), c["name"]
        return
    meta, lg, ids, w = kept
    assert meta.tolist() == c["cap_meta"].tolist(), (c["name"], meta, c["cap_meta"])
    assert np.array_equal(lg, c["cap_lg"][:c["E"]]) and np.array_equal(ids, c["cap_ids"]) and \
        np.array_equal(w.astype(np.float32), c["cap_w"])


@pytest.mark.parametrize("mistake", ["bias_dropped", "one_expert_group_score", "no_renorm"])
def test_planted_mistakes_fail(monkeypatch, mistake):
    orig_judge = R.judge
    if mistake == "one_expert_group_score":
        monkeypatch.setattr(R, "_group_scores", lambda g, biased: g.max(-1))
    else:
        def wrong(lf, kid, kw, k, scoring, renormalize, bias, groups, topk_group, scale, u):
            if mistake == "bias_dropped":
                bias = None
            else:
                renormalize = False
            return orig_judge(lf, kid, kw, k, scoring, renormalize, bias, groups, topk_group, scale, u)
        monkeypatch.setattr(R, "judge", wrong)
    mismatched = 0
    for i in range(len(NAMES)):
        c = route_case(i)
        sb, wb, _ = R.judge(c["logits"], c["ids"], c["w"], c["k"], c["scoring"], c["renorm"], c["bias"],
                            c["groups"], c["tg"], c["scale"], R.unit_roundoff(c["dt"]))
        mismatched += not (np.array_equal(sb, c["set_bad"]) and np.array_equal(wb, c["w_bad"]))
    assert mismatched > 0, mistake
