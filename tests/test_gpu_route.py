"""The MoE router check on the GPU (sdc_route_check through serve_route) against the reference's answers
(tests/golden/route.npz: route_check_torch's state row and kept row for 165 seeded calls, serve_route.judge on every
row) and against the oracle (oracle/route.py) on router calls of real models' shapes.

The state rows are integer counts and packed keys: compared exactly; the worst weight difference (float bits) to
1e-6 of the weights' size plus 3e-7 (exp in another library).  The kept row is one of the sampled rows the call found
wrong (the two samples race for it on the GPU; the reference keeps the first): its logits, ids and weights exactly."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import route as R
from tests.test_oracle_route import NAMES, route_case

pytestmark = pytest.mark.gpu

TDT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def state_problems(got, want, wmax: float) -> list:
    """Columns of a state row that differ: counts and packed keys exactly, the worst weight difference to 1e-6 of
    the largest weight plus 3e-7 (a few float32 ulps of the weights: exp computed by another library)."""
    bad = []
    for col in range(R.COLS):
        a, b = int(got[col]), int(want[col])
        if col == R.C_WDIFF:
            fa, fb = (float(np.array([v & R.M32], np.uint32).view(np.float32)[0]) for v in (a, b))
            if abs(fa - fb) > 1e-6 * wmax + 3e-7:
                bad.append((col, fa, fb))
        elif a != b:
            bad.append((col, a, b))
    return bad


def _bufs(rows: int, e: int, k: int):
    from sdcguard_amd import serve_route as sr
    return (torch.zeros(rows, sr.COLS, dtype=torch.int64, device="cuda"),
            torch.zeros(rows, sr.CAP_COLS, dtype=torch.int64, device="cuda"),
            torch.zeros(rows, e, device="cuda"), torch.zeros(rows, k, dtype=torch.int64, device="cuda"),
            torch.zeros(rows, k, device="cuda"))


def _word(v: int) -> torch.Tensor:
    return torch.tensor([v], dtype=torch.int64, device="cuda")


def _dev_case(c):
    if c["bits"] is None:
        lg = torch.from_numpy(c["logits"]).cuda()
    else:
        lg = torch.from_numpy(c["bits"].astype(np.uint16).view(np.int16)).cuda().view(TDT[c["dt"]])
        lg = lg.reshape(c["bits"].shape)
    bias = None if c["bias"] is None else torch.from_numpy(c["bias"]).cuda()
    return lg, torch.from_numpy(c["w"]).cuda(), torch.from_numpy(c["ids"]).cuda(), bias


def _call(c, lg, w, ids, bias, real, step, nl, idx, bufs, slot=0):
    from sdcguard_amd import serve_route as sr
    st, meta, clg, cid, cw = bufs
    sr.route_check(lg, w, ids, c["k"], c["scoring"], c["renorm"], bias, c["groups"], c["tg"], c["scale"],
                   _word(real), _word(step), st, slot, nl, idx, meta, clg, cid, cw)


def _kept_ok(c, meta, clg, cid, cw, logits, ids, w, bad: list, kinds: dict) -> list:
    """What is wrong with a kept row (an empty list: nothing)."""
    out = []
    meta = [int(v) for v in meta]
    if not bad:
        return [] if not any(meta) else [("kept a row of a clean call", meta)]
    if meta[0] != 1 or meta[1] not in bad:
        return [("kept", meta, "bad rows", bad)]
    r = meta[1]
    want_code = {"fp32": 0, "bf16": 1, "fp16": 2}[c["dt"]]
    if meta[2:] != [c["step"] & R.M32, kinds[r], c["E"], want_code]:
        out.append(("meta", meta, kinds[r], c["E"], want_code))
    if not np.array_equal(clg[:c["E"]], logits[r]) or not np.array_equal(cid[:c["k"]], ids[r].astype(np.int64)) or \
            not np.array_equal(cw[:c["k"]], w[r].astype(np.float32)):
        out.append(("kept data", r))
    return out


@pytest.mark.parametrize("i", range(len(NAMES)))
def test_call_matches_reference(i):
    """One router call as the reference's route_check_torch made it (step 5 of routers taking turns 2 ways, this one
    index 1; inactive and no-row cases included): the state row and the kept row."""
    c = route_case(i)
    print(c["name"], flush=True)
    lg, w, ids, bias = _dev_case(c)
    bufs = _bufs(1, c["E"], c["k"])
    _call(c, lg, w, ids, bias, c["real"], c["step"], c["nl"], c["idx"], bufs)
    st = bufs[0][0].cpu().numpy()
    probs = state_problems(st, c["state"], float(np.abs(c["w"]).max()))
    assert not probs, (c["name"], probs)
    rows = R.sample_rows(c["step"], min(c["real"], 8), c["nl"])
    live = c["real"] > 0 and c["step"] % c["nl"] == c["idx"]
    bad = [int(r) for r in rows if live and (c["set_bad"][r] or c["w_bad"][r]) and not (c["ids"][r] == -1).all()]
    kinds = {int(r): (R.KIND_SET if c["set_bad"][r] else R.KIND_WEIGHT) for r in rows}
    probs = _kept_ok(c, bufs[1][0].cpu().numpy(), bufs[2][0].cpu().numpy(), bufs[3][0].cpu().numpy(),
                     bufs[4][0].cpu().numpy(), c["logits"], c["ids"], c["w"], bad, kinds)
    assert not probs, (c["name"], probs)


@pytest.mark.parametrize("i", range(len(NAMES)))
def test_every_row_judged_as_the_reference_judges_it(i):
    """Each row of the call alone (a one-row call: both samples are the row, each finding counts twice): the
    reference's judge on every row, the wrong sets and wrong weights exactly, the worst weight difference."""
    c = route_case(i)
    print(c["name"], flush=True)
    lg, w, ids, bias = _dev_case(c)
    m = lg.shape[0]
    bufs = _bufs(m, c["E"], c["k"])
    for r in range(m):
        _call(c, lg[r:r + 1], w[r:r + 1], ids[r:r + 1], bias, 1, 0, 1, 0, bufs, slot=r)
    st = bufs[0].cpu().numpy()
    for r in range(m):
        pad = bool((c["ids"][r] == -1).all())
        want = [1, 0 if pad else 2 * int(c["set_bad"][r]), 0 if pad else 2 * int(c["w_bad"][r]), 0 if pad else 2]
        got = [int(st[r, R.C_CALLS]), int(st[r, R.C_SET]), int(st[r, R.C_WEIGHT]), int(st[r, R.C_ROWS])]
        assert got == want, (c["name"], r, got, want)
        if not pad:
            wd = float(np.array([st[r, R.C_WDIFF] & R.M32], np.uint32).view(np.float32)[0])
            ref = float(c["diff"][r].max())
            assert abs(wd - ref) <= 1e-6 * float(np.abs(c["w"][r]).max()) + 3e-7, (c["name"], r, wd, ref)


# ------------------------------------------------------------------------------ router calls of real models' shapes
# name: (experts, k, scoring, renormalize, bias, groups, topk_group, scale, logits dtype, rows)
MODELS = {
    "mixtral_top2_of_8": (8, 2, 0, True, False, 0, 0, 1.0, torch.bfloat16, 4096),
    "qwen3_top8_of_128": (128, 8, 0, True, False, 0, 0, 1.0, torch.bfloat16, 4096),
    "llama4_sigmoid_top1_of_16": (16, 1, 1, False, False, 0, 0, 1.0, torch.bfloat16, 2048),
    "deepseek_v3_grouped": (256, 8, 1, True, True, 8, 4, 2.5, torch.bfloat16, 8192),
    "deepseek_v2_lite_grouped_softmax": (64, 6, 0, False, False, 1, 1, 1.0, torch.float16, 2048),
    "glm_sigmoid_biased_top8_of_160": (160, 8, 1, True, True, 0, 0, 2.5, torch.float32, 1024),
    "widest_top32_of_2048": (2048, 32, 0, True, False, 16, 4, 1.0, torch.float32, 512),
}


def _router(lg: torch.Tensor, k, scoring, renorm, bias, groups, tg, scale):
    """A router's result (the role vLLM's fused top-k kernels play): fp32 scores, groups, top-k, weights."""
    s = torch.softmax(lg.float(), -1) if scoring == 0 else torch.sigmoid(lg.float())
    ch = s + bias if bias is not None else s
    if groups:
        m, e = ch.shape
        g = ch.view(m, groups, e // groups)
        gs = g.topk(2, -1).values.sum(-1) if bias is not None else g.amax(-1)
        keep = torch.zeros(m, groups, dtype=torch.bool, device=ch.device).scatter(1, gs.topk(tg, -1).indices, True)
        ch = ch.masked_fill(~keep.repeat_interleave(e // groups, 1), float("-inf"))
    ids = ch.topk(k, -1).indices
    w = s.gather(1, ids)
    if renorm:
        w = w / w.sum(-1, keepdim=True)
    return (w * scale).float(), ids.to(torch.int32)


def _model_case(name: str, seed: int = 0):
    e, k, scoring, renorm, has_bias, groups, tg, scale, dt, m = MODELS[name]
    g = torch.Generator(device="cuda").manual_seed(seed)
    lg = (torch.randn(m, e, device="cuda", generator=g) * 2).to(dt)
    bias = (torch.randn(e, device="cuda", generator=g) * 0.03) if has_bias else None
    w, ids = _router(lg, k, scoring, renorm, bias, groups, tg, scale)
    c = {"k": k, "scoring": scoring, "renorm": renorm, "groups": groups, "tg": tg, "scale": scale, "E": e,
         "dt": {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}[dt]}
    return c, lg, w, ids, bias


def _oracle_state(c, lg, w, ids, bias, real, steps, nl, idx):
    st = None
    npb = None if bias is None else bias.cpu().numpy()
    lgn, wn, idn = lg.float().cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy()
    for s in steps:
        st, _ = R.route_check(lgn, wn, idn, c["k"], c["scoring"], c["renorm"], npb, c["groups"], c["tg"], c["scale"],
                              c["dt"], real, s, nl, idx, state=st)
    return st


@pytest.mark.parametrize("name", list(MODELS))
def test_model_shapes_match_oracle_over_many_steps(name):
    """48 steps of one of 3 routers (index 2) over the real rows of a padded batch: the state row the oracle gives,
    clean routing (no finding) and, after a row's expert and another row's weight are changed, the findings."""
    c, lg, w, ids, bias = _model_case(name)
    m = lg.shape[0]
    real = m - 37
    steps = list(range(2, 2 + 3 * 48))
    print(name, tuple(lg.shape), lg.dtype, flush=True)
    for planted in (False, True):
        if planted:
            e, k = c["E"], c["k"]
            s_hit = [(s // 3 * R.ROW_A) % real for s in steps if s % 3 == 2][:6]
            r_set, r_w = s_hit[1], s_hit[4]
            worst = lg[r_set].float().argmin()
            ids = ids.clone()
            w = w.clone()
            ids[r_set, -1] = worst.to(torch.int32) if int(worst) not in ids[r_set].tolist() else \
                (ids[r_set, -1] + e // 2) % e
            w[r_w, 0] *= 1.05
        bufs = _bufs(1, c["E"], c["k"])
        for s in steps:
            _call(c, lg, w, ids, bias, real, s, 3, 2, bufs)
        got = bufs[0][0].cpu().numpy()
        want = _oracle_state(c, lg, w, ids, bias, real, steps, 3, 2)
        print(planted, got.tolist(), want.tolist(), flush=True)
        probs = state_problems(got, want, float(w.abs().max()))
        assert not probs, (name, planted, probs)
        assert got[R.C_CALLS] == 48 and got[R.C_ROWS] == 96
        if not planted:
            assert got[R.C_SET] == 0 and got[R.C_WEIGHT] == 0
        else:
            assert got[R.C_SET] >= 1 and got[R.C_WEIGHT] >= 1


@pytest.mark.parametrize("name", ["qwen3_top8_of_128", "llama4_sigmoid_top1_of_16", "deepseek_v3_grouped"])
@pytest.mark.parametrize("fault", ["expert", "weight"])
def test_wrong_expert_or_weight_is_located(name, fault):
    """One row's routing changed (an expert swapped for the row's worst-scoring one, or one weight 5% off: bf16
    logits allow 2.4%): at the
    step that samples the row, the finding's kind, step and row; the kept row holds it; the other steps are clean."""
    from sdcguard_amd import serve_route as sr
    c, lg, w, ids, bias = _model_case(name, seed=3)
    m = lg.shape[0]
    step = 1234
    row = (step * R.ROW_A) % m                        # the first sample of `step` (one router: nlayers 1)
    ids, w = ids.clone(), w.clone()
    if fault == "expert":
        cand = [int(v) for v in lg[row].float().argsort().tolist() if int(v) not in ids[row].tolist()]
        ids[row, -1] = cand[0]
    else:
        w[row, 0] *= 1.05
    bufs = _bufs(1, c["E"], c["k"])
    for s in (step - 1, step, step + 1):
        _call(c, lg, w, ids, bias, m, s, 1, 0, bufs)
    st = bufs[0][0].cpu().tolist()
    meta = bufs[1][0].cpu().tolist()
    kind = sr.KIND_SET if fault == "expert" else sr.KIND_WEIGHT
    print(name, fault, row, st, meta, flush=True)
    assert st[sr.C_CALLS] == 3 and st[sr.C_ROWS] == 6
    assert (st[sr.C_SET], st[sr.C_WEIGHT]) == ((1, 0) if fault == "expert" else (0, 1))
    assert st[sr.C_LAST] == ((step & 0x7FFFFFFF) << 32) | (kind << 24) | row
    assert meta == [1, row, step, kind, c["E"], sr.DTYPE_CODE[lg.dtype]]
    assert torch.equal(bufs[2][0, :c["E"]], lg[row].float())
    assert torch.equal(bufs[3][0, :c["k"]], ids[row].long()) and torch.equal(bufs[4][0, :c["k"]], w[row])


def test_refused_cases_raise_before_any_launch():
    from sdcguard_amd import _lib, serve_route as sr
    c, lg, w, ids, bias = _model_case("qwen3_top8_of_128")
    bufs = _bufs(1, 4096, 64)
    st, meta, clg, cid, cw = bufs
    with pytest.raises(_lib.HipLibraryError):          # 3 groups do not divide 128 experts
        sr.route_check(lg, w, ids, 8, 0, True, None, 3, 1, 1.0, _word(10), _word(0), st, 0, 1, 0, meta, clg, cid, cw)
    wide = torch.zeros(4, 4096, device="cuda")
    with pytest.raises(_lib.HipLibraryError):          # more than 2048 experts
        sr.route_check(wide, w[:4], ids[:4], 8, 0, True, None, 0, 0, 1.0, _word(4), _word(0), st, 0, 1, 0, meta,
                       clg, cid, cw)
    with pytest.raises(ValueError):                    # a kept-row buffer narrower than the experts
        sr.route_check(lg, w, ids, 8, 0, True, None, 0, 0, 1.0, _word(10), _word(0), st, 0, 1, 0, meta,
                       clg[:, :64], cid, cw)
    torch.cuda.synchronize()
    assert not st.any()


# ------------------------------------------------------------------------------------------- the serving flow
def _fake_router(kind: str, **attrs):
    cls = type(kind, (), {})
    r = cls()
    for k, v in attrs.items():
        setattr(r, k, v)
    return r


def _deepseek_router(bias):
    return _fake_router("GroupedTopKRouter", top_k=8, global_num_experts=256, scoring_func="sigmoid",
                        renormalize=True, e_score_correction_bias=bias, routed_scaling_factor=2.5,
                        num_expert_group=8, topk_group=4)


def test_route_checks_serving_flow():
    """ServeGuard.route_checks(): two routers (a grouped DeepSeek one, a softmax top-8 one) take turns; clean steps
    raise nothing; a wrong expert at a step that samples its row is reported with its step and row and the recheck
    finds the kept row wrong again; a wrong weight likewise."""
    from sdcguard_amd.serve import ServeGuard
    from sdcguard_amd import serve_route as sr
    c1, lg1, w1, ids1, bias1 = _model_case("deepseek_v3_grouped", seed=5)
    c2, lg2, w2, ids2, _ = _model_case("qwen3_top8_of_128", seed=6)
    r1 = _deepseek_router(bias1)
    r2 = _fake_router("FusedTopKRouter", top_k=8, global_num_experts=128, scoring_func="softmax", renormalize=True)
    g = ServeGuard()
    rc = g.route_checks()
    assert rc.add(r1, "layers.3.mlp.router", "cuda") == 0 and rc.add(r2, "layers.4.mlp.router", "cuda") == 1
    assert rc.finalize() == 2
    real = 1000

    def step(s, lg_a=lg1, w_a=w1, ids_a=ids1, lg_b=lg2, w_b=w2, ids_b=ids2):
        g.mark_step(s, real)
        sr.check_call(r1._sdcguard_route, lg_a, w_a, ids_a)
        sr.check_call(r2._sdcguard_route, lg_b, w_b, ids_b)
        g.end_step()

    for s in range(1, 9):
        step(s)
    assert g.poll(wait=True) == [] and rc.stats["calls"] == 8 and rc.stats["rows"] == 16
    assert rc.coverage()["layers_checked"] == 2 and rc.coverage()["never_checked"] == []
    # router 1 is on turn at even steps; at step 20 its first sample is row (20 // 2 * 7919) % real
    row = (10 * R.ROW_A) % real
    bad_ids = ids1.clone()
    cand = [int(v) for v in lg1[row].float().argsort().tolist() if int(v) not in ids1[row].tolist()]
    bad_ids[row, 0] = cand[0]
    step(19)
    step(20, ids_a=bad_ids)
    ev = g.poll(wait=True)
    print([e.extra for e in ev], flush=True)
    assert len(ev) == 1 and ev[0].detector == "serve_route" and ev[0].layer == "layers.3.mlp.router"
    d = ev[0].extra
    assert d["finding"] == "wrong_experts" and d["captured"] == {"step": 20, "row": row}
    assert d["recheck"]["verdict"] == "output_wrong" and d["recheck"]["captured"]["row"] == row
    assert d["policy"]["groups"] == 8 and d["policy"]["bias"] is True
    # router 2 (odd steps) at step 31: row (31 // 2 * 7919) % real, one weight 10% off (bf16 logits allow
    # 1e-4 + 6 u = 2.4% of a weight)
    row2 = (15 * R.ROW_A) % real
    bad_w = w2.clone()
    bad_w[row2, 3] *= 1.10
    step(31, w_b=bad_w)
    ev = g.poll(wait=True)
    assert len(ev) == 1 and ev[0].layer == "layers.4.mlp.router"
    d = ev[0].extra
    assert d["finding"] == "wrong_weights" and d["captured"]["row"] == row2 and d["worst_weight_difference"] > 1e-4
    assert d["recheck"]["verdict"] == "output_wrong"
    g.detach()
    assert getattr(r1, "_sdcguard_route", None) is None


def test_route_check_in_a_captured_graph():
    """The check captured once with a router call and replayed at 6 steps (the step word written before each
    replay, eager work and a synchronization between replays): the counts of the eager calls, replay after replay,
    and a wrong row planted in the graph's input found at the step that samples it."""
    from sdcguard_amd.serve import ServeGuard
    from sdcguard_amd import serve_route as sr
    c, lg, w, ids, bias = _model_case("deepseek_v3_grouped", seed=7)
    r = _deepseek_router(bias)
    g = ServeGuard()
    rc = g.route_checks()
    rc.add(r, "router", "cuda")
    rc.finalize()
    real = 3000
    g.mark_step(0, real)
    sr.check_call(r._sdcguard_route, lg, w, ids)         # (warm-up outside the graph)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            sr.check_call(r._sdcguard_route, lg, w, ids)
    torch.cuda.current_stream().wait_stream(s)
    g.poll(wait=True)
    base = rc.stats["calls"]
    for i, st in enumerate(range(100, 106)):
        g.mark_step(st, real)
        graph.replay()
        g.end_step()
        torch.cuda.synchronize()
        _ = (lg.float() * 2).sum()                       # eager work between replays
        torch.cuda.synchronize()
        assert g.poll(wait=True) == []
        assert rc.stats["calls"] == base + i + 1 and rc.stats["rows"] == 2 * (base + i + 1)
    row = (200 * R.ROW_A) % real
    cand = [int(v) for v in lg[row].float().argsort().tolist() if int(v) not in ids[row].tolist()]
    ids[row, 2] = cand[0]                               # in place: the graph reads this tensor
    g.mark_step(200, real)
    graph.replay()
    g.end_step()
    ev = g.poll(wait=True)
    assert len(ev) == 1 and ev[0].extra["captured"] == {"step": 200, "row": row}
    g.detach()
