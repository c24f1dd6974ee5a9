"""The sampled fused-MoE recompute on the GPU (sdc_moe_check through serve_moe) against the reference's state and
kept rows (tests/golden/moe.npz), the oracle on larger layers (every output's score), located faults, and the
MoEChecks flow (turns, routing alerts, output alerts with the kept row rechecked, graph capture).

Tolerances as the oracle's own test: counts, located faults and the kept row exactly; scores to 0.3 + 2% (the
recompute's fp32 sums run in another order than the reference's)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import serve_moe as om
from tests.test_oracle_moe import NAMES, agrees, moe_case, run_oracle

pytestmark = pytest.mark.gpu


def _dev_words(w, dt):
    t = torch.from_numpy(np.ascontiguousarray(w).view(np.int16))
    return t.view(torch.bfloat16 if dt == "bf16" else torch.float16).cuda()


def _run_gpu(c, x=None, y=None, scores=None):
    from sdcguard_amd import serve_moe as sm
    dt = c["dt"]
    x = _dev_words(c["xw"], dt) if x is None else x
    y = _dev_words(c["yw"], dt) if y is None else y
    w13, w2 = _dev_words(c["w13w"], dt), _dev_words(c["w2w"], dt)
    ids = torch.from_numpy(c["ids"]).cuda()
    g = torch.from_numpy(c["g"]).cuda()
    emap = None if c["emap"] is None else torch.from_numpy(c["emap"]).cuda()
    H, k = x.shape[1], c["k"]
    st = torch.zeros(1, sm.COLS, dtype=torch.int64, device="cuda")
    cm = torch.zeros(1, sm.CAP_COLS, dtype=torch.int32, device="cuda")
    cx, cy = torch.zeros(1, H, device="cuda"), torch.zeros(1, H, device="cuda")
    ci, cg = torch.zeros(1, max(k, 8), dtype=torch.int64, device="cuda"), torch.zeros(1, max(k, 8), device="cuda")
    sb = torch.full((1,), c["raw"], dtype=torch.int64, device="cuda")
    sm.moe_check(x, y, g, ids, w13, w2, emap, c["act"], c["rf"], st, 0, sb, c["nl"], c["idx"], cm, cx, cy, ci, cg,
                 sm.MOE_Z, scores_out=scores)
    cap = {"meta": cm[0].cpu().numpy().astype(np.int64), "x": cx[0].cpu().numpy(), "y": cy[0].cpu().numpy(),
           "ids": ci[0, :k].cpu().numpy(), "g": cg[0, :k].cpu().numpy()}
    return st[0].cpu().numpy(), cap


@pytest.mark.parametrize("i", range(len(NAMES)))
def test_state_and_kept_row_match_reference(i):
    c = moe_case(i)
    print(c["name"], flush=True)
    st, cap = _run_gpu(c)
    bad = agrees(st, cap, c)
    assert not bad, (c["name"], bad)


@pytest.mark.parametrize("dt,act,rf", [("bf16", 0, False), ("fp16", 1, True), ("bf16", 1, False)])
def test_larger_layer_scores_against_oracle_and_faults(dt, act, rf):
    """64 experts of 1024 x 512 (2I x H = 1024 x 1024... H 1024, I 512), top 8, 96 rows: every output's score
    against the oracle; then another row's output in a sampled row, one expert's output missing, and a NaN: each
    over the line at its row, the kept row that row."""
    g0 = torch.Generator().manual_seed(7 + act)
    E, H, I, K, M = 64, 1024, 512, 8, 96
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    w13 = (torch.randn(E, 2 * I, H, generator=g0) * 0.03).to(tdt)
    w2 = (torch.randn(E, H, I, generator=g0) * 0.03).to(tdt)
    x = torch.randn(M, H, generator=g0).to(tdt)
    gw, ids = torch.topk(torch.softmax(torch.randn(M, E, generator=g0), -1), K, -1)
    ids = ids.to(torch.int32)
    step, nl, idx = 11, 3, 2
    raw = (80 << 32) | step
    rows = om.sample_rows(step, 80, nl)
    xs = x.float().numpy()
    r_all, *_ = om.recompute(xs, ids.numpy(), gw.numpy(), w13.float().numpy(), w2.float().numpy(), None, act, rf, dt)
    y = torch.from_numpy(r_all).to(tdt)
    c = dict(name=f"{dt}_{act}", x=xs, y=y.float().numpy(), xw=x.view(torch.int16).numpy(),
             yw=y.view(torch.int16).numpy(), w13=w13.float().numpy(), w2=w2.float().numpy(),
             w13w=w13.view(torch.int16).numpy(), w2w=w2.view(torch.int16).numpy(), ids=ids.numpy(), g=gw.numpy(),
             emap=None, act=act, rf=rf, raw=raw, nl=nl, idx=idx, dt=dt, k=K)
    zs = torch.zeros(2, H, device="cuda")
    st, cap = _run_gpu(c, scores=zs)
    _, _, oz = run_oracle(c)
    got = zs.cpu().numpy()
    diff = np.abs(got - oz)
    print(f"{dt} act {act}: max z {got.max():.3f} (oracle {oz.max():.3f}), max |dz| {diff.max():.3f}")
    assert (diff <= 0.3 + 0.02 * np.abs(oz)).all() and got.max() < 3
    assert st[om.C_CALLS] == 1 and st[om.C_ROWS] == 2 and st[om.C_UNJ] == 0
    for what in ("other_row", "missing_expert", "nan"):
        y2 = y.clone()
        r0 = rows[0]
        if what == "other_row":
            y2[r0] = y[(r0 + 1) % M]
        elif what == "missing_expert":
            ids2 = ids.clone()
            ids2[r0, 3] = (ids2[r0, 3] + 1) % E
            r_bad, *_ = om.recompute(xs[r0:r0 + 1], ids2[r0:r0 + 1].numpy(), gw[r0:r0 + 1].numpy(),
                                     w13.float().numpy(), w2.float().numpy(), None, act, rf, dt)
            y2[r0] = torch.from_numpy(r_bad[0]).to(tdt)
        else:
            y2[r0, 77] = float("nan")
        c2 = dict(c, yw=y2.view(torch.int16).numpy(), y=y2.float().numpy())
        st2, cap2 = _run_gpu(c2)
        z = float(np.array([int(st2[0]) >> 32], np.uint32).view(np.float32)[0])
        assert z > 6 and int(st2[0]) & 0xFFFFFFFF == r0 and cap2["meta"][0] == 1 and cap2["meta"][1] == r0, \
            (what, z, int(st2[0]) & 0xFFFFFFFF, r0, cap2["meta"])
        st3, cap3, _ = run_oracle(c2)
        assert not agrees(st2, cap2, dict(c2, state=st3, cap=cap3["meta"], cap_x=cap3["x"], cap_y=cap3["y"],
                                          cap_ids=cap3["ids"], cap_g=cap3["g"])), what


def test_out_of_range_expert_ids_are_counted_not_read():
    """Expert ids a router cannot produce (past the experts held, past the expert map, below -1) are never used to
    index the weights: a sampled row holding one disagrees with its output (its slot adds nothing), and every known
    real row holding one is counted with the rows missing experts."""
    g0 = torch.Generator().manual_seed(3)
    E, H, I, K, M = 8, 256, 128, 2, 24
    w13 = (torch.randn(E, 2 * I, H, generator=g0) * 0.05).bfloat16()
    w2 = (torch.randn(E, H, I, generator=g0) * 0.05).bfloat16()
    x = torch.randn(M, H, generator=g0).bfloat16()
    gw, ids = torch.topk(torch.softmax(torch.randn(M, E, generator=g0), -1), K, -1)
    ids = ids.to(torch.int32)
    step, nl, idx = 5, 1, 0
    raw = (20 << 32) | step
    r0 = int(om.sample_rows(step, 20, nl)[0])
    r_all, *_ = om.recompute(x.float().numpy(), ids.numpy(), gw.numpy(), w13.float().numpy(), w2.float().numpy(),
                             None, 0, False, "bf16")
    y = torch.from_numpy(r_all).bfloat16()
    base = dict(name="oob", xw=x.view(torch.int16).numpy(), yw=y.view(torch.int16).numpy(),
                w13w=w13.view(torch.int16).numpy(), w2w=w2.view(torch.int16).numpy(), g=gw.numpy(), act=0, rf=False,
                raw=raw, nl=nl, idx=idx, dt="bf16", k=K)
    bad = ids.clone()
    bad[r0, 1] = 1 << 30                                  # the sampled row: an id far past the 8 experts
    bad[(r0 + 3) % 20, 0] = E                             # another real row: the first id past the end
    bad[21, 0] = -7                                       # a row past the real ones: not scanned
    st, _ = _run_gpu(dict(base, ids=bad.numpy(), emap=None))
    z = float(np.array([int(st[0]) >> 32], np.uint32).view(np.float32)[0])
    print("no map:", z, st.tolist())
    assert z > 6 and int(st[0]) & 0xFFFFFFFF == r0
    assert st[om.C_PARTIAL] == 2 and st[om.C_UNROUTED] == 0 and st[om.C_BADROW] & 0xFFFFFFFF == max(r0, (r0 + 3) % 20) + 1
    # with an expert map of 12 global ids (the last four on another GPU): 12 is out of range, 11 is not
    emap = np.array(list(range(E)) + [-1, -1, -1, -1], np.int32)
    ok = ids.clone()
    ok[(r0 + 1) % 20, 0] = 11                             # another GPU's expert: a valid routing
    ok[(r0 + 2) % 20, 1] = 12
    st2, _ = _run_gpu(dict(base, ids=ok.numpy(), emap=emap))
    print("map:", st2.tolist())
    assert st2[om.C_PARTIAL] == 1 and st2[om.C_UNROUTED] == 0


class _Act:
    value = "silu"


class _Backend:
    name = "TRITON"


class UnquantizedFusedMoEMethod:
    unquantized_backend = _Backend()


class _FusedMoE(torch.nn.Module):
    """A stand-in for a serving stack's fused MoE layer (the attributes describe() reads)."""

    def __init__(self, E=16, H=512, I=256, K=4, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.w13_weight = torch.nn.Parameter((torch.randn(E, 2 * I, H, generator=g) * 0.04).bfloat16().cuda(),
                                             requires_grad=False)
        self.w2_weight = torch.nn.Parameter((torch.randn(E, H, I, generator=g) * 0.04).bfloat16().cuda(),
                                            requires_grad=False)
        self.quant_method = UnquantizedFusedMoEMethod()
        self.activation = _Act()
        self.top_k = K
        self.E = E

    def run(self, x, gen):
        from sdcguard_amd import serve_moe as sm
        gw, ids = torch.topk(torch.softmax(torch.randn(x.shape[0], self.E, generator=gen), -1), self.top_k, -1)
        gw, ids = gw.cuda(), ids.to(torch.int32).cuda()
        y = torch.from_numpy(om.recompute(x.float().cpu().numpy(), ids.cpu().numpy(), gw.cpu().numpy(),
                                          self.w13_weight.float().cpu().numpy(), self.w2_weight.float().cpu().numpy(),
                                          None, 0, False, "bf16")[0]).bfloat16().cuda()
        return gw, ids, y


def test_moechecks_flow_alerts_and_capture():
    from sdcguard_amd import serve_moe as sm
    seen = []

    class _G:
        on_alert = staticmethod(seen.append)

    mc = sm.MoEChecks(_G())
    layers = [_FusedMoE(seed=s) for s in range(3)]
    for i, L in enumerate(layers):
        assert mc.add(L, f"moe{i}") == i
    q = _FusedMoE(seed=9)
    q.quant_method = object()
    assert mc.add(q, "quantized") is None and "quantized" in mc.unsupported
    assert mc.finalize() == 3
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(24, 512, generator=gen).bfloat16().cuda()
    calls = [(L, *L.run(x, gen)) for L in layers]
    for step in range(6):                             # each layer active every third step: all clean
        mc.mark_step(step, 20)
        for L, gw, ids, y in calls:
            sm.check_call(L._sdcguard_moe, x, gw, ids, y)
        mc.end_step()
    assert mc.poll(wait=True) == [] and mc.stats["active_calls"] == 6 and mc.stats["rows_checked"] == 12
    # layer 1 at step 7: a sampled row's output replaced by another row's; a real row unrouted in layer 2 at step 8
    L1, gw1, ids1, y1 = calls[1]
    r0 = om.sample_rows(7, 20, 3)[0]
    bad = y1.clone()
    bad[r0] = y1[(r0 + 5) % 24]
    mc.mark_step(7, 20)
    sm.check_call(L1._sdcguard_moe, x, gw1, ids1, bad)
    mc.end_step()
    L2, gw2, ids2, y2 = calls[2]
    ids_bad = ids2.clone()
    ids_bad[4] = -1
    mc.mark_step(8, 20)
    sm.check_call(L2._sdcguard_moe, x, gw2, ids_bad, y2)
    mc.end_step()
    ev = mc.poll(wait=True)
    kinds = {e.layer: e.extra["kind"] for e in ev}
    print(kinds, [e.extra.get("recheck", {}).get("verdict") for e in ev])
    assert kinds == {"moe1": "moe_experts", "moe2": "moe_routing"}, kinds
    e1 = next(e for e in ev if e.layer == "moe1")
    assert e1.extra["row"] == r0 and e1.extra["recheck"]["verdict"] == "output_wrong" and \
        e1.extra["weights_changed_since_load"] is False and e1.extra["captured"]["row"] == r0
    e2 = next(e for e in ev if e.layer == "moe2")
    assert e2.extra["finding"] == "real_rows_unrouted" and e2.extra["row"] == 4
    # a changed expert weight: the recheck agrees with the (changed) weights, and says they changed since load
    r10 = om.sample_rows(10, 20, 3)[0]                 # (a row layer 1 samples at step 10)
    ex = int(ids1[r10, 0])
    with torch.no_grad():
        L1.w2_weight[ex].mul_(2)
    mc.mark_step(10, 20)
    sm.check_call(L1._sdcguard_moe, x, gw1, ids1, y1)
    mc.end_step()
    ev = mc.poll(wait=True)
    assert len(ev) == 1 and ev[0].extra["weights_changed_since_load"] is True, ev
    with torch.no_grad():
        L1.w2_weight[ex].div_(2)
    # the calls captured in a graph: replays count as eager calls do
    st = mc.tables[layers[0].w13_weight.device].state
    mc.mark_step(12, 20)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for L, gw, ids, y in calls:
            sm.check_call(L._sdcguard_moe, x, gw, ids, y)
        torch.cuda.synchronize()
        st.zero_()
        with torch.cuda.graph(graph, stream=s):
            for L, gw, ids, y in calls:
                sm.check_call(L._sdcguard_moe, x, gw, ids, y)
    torch.cuda.synchronize()
    st.zero_()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert int(st[:, om.C_CALLS].sum()) == 1 and int(st[:, om.C_ROWS].sum()) == 2, (rep, st)
        z = np.array([int(v) >> 32 for v in st[:, 0].tolist()], np.uint32).view(np.float32)
        assert (z < 6).all(), z
        _ = (x.float() * 2).sum().item()
        st.zero_()
    mc.end_step()
    mc.detach()


def test_serveguard_reaches_fp8_and_moe_checks():
    """ServeGuard.fp8_checks() / moe_checks(): mark_step, end_step and poll of the guard reach both."""
    from sdcguard_amd import serve_fp8 as sf
    from sdcguard_amd import serve_moe as sm
    from sdcguard_amd.serve import ServeGuard
    from tests.test_gpu_fp8 import _Quant
    seen = []
    g = ServeGuard(on_alert=seen.append)
    L = _FusedMoE(seed=3)
    mc = g.moe_checks()
    assert mc.add(L, "experts") == 0 and mc.finalize() == 1
    lin = torch.nn.Linear(64, 64)
    a = g.fp8_checks().add(lin, "fp8", _Quant(), None, torch.device("cuda", 0))
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(16, 512, generator=gen).bfloat16().cuda()
    gw, ids, y = L.run(x, gen)
    xf = torch.randn(16, 64, device="cuda").bfloat16()
    s_ok = (xf.float().abs().amax() / 448.0).reshape(1)
    g.mark_step(4, 16)
    sf.check_call(a, xf, sf.quantize(xf, s_ok * 1.5, False), s_ok * 1.5)      # a wrong per-tensor scale
    bad = y.clone()
    bad[om.sample_rows(4, 16, 1)[0]] += 1.0                                   # a wrong expert output
    sm.check_call(L._sdcguard_moe, x, gw, ids, bad)
    g.end_step()
    ev = g.poll(wait=True)
    assert sorted(e.detector for e in ev) == ["serve_fp8", "serve_moe"], ev
    assert len(seen) == 2
    g.detach()
