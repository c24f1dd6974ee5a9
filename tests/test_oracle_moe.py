"""The sampled fused-MoE recompute oracle (oracle/serve_moe.py) against the reference's state rows and kept rows
(tests/golden/moe.npz, serve_moe.moe_check_torch on its verification scenarios).

Counts (active calls, rows checked, unjudged outputs, unrouted and partly routed real rows, the last such row),
located faults (row and column of a score over the line) and the kept row (flag, row, step, input, output, experts,
weights) exactly; scores to 0.3 + 2% (the recompute's matmuls sum in another order than torch's on the CPU, which
moves a rounded intermediate by a step at a boundary: the bound's flip term).  A planted mistake (the routing weight
not applied) must fail."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import serve_moe as om
from tests import _golden as G

MO = G.load("moe.npz")
NAMES = G.names(MO)


def _f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", int(bits) & 0xFFFFFFFF))[0]


def moe_case(i):
    p = f"c{i}_"
    ids = [str(v) for v in MO[p + "ids"]]
    is16, act, rf, raw, nl, idx, has_map = (int(v) for v in MO[p + "meta"])
    dt = "fp16" if is16 else "bf16"
    topk = MO[p + "topk"]
    k = topk.shape[1]
    w13w, w2w = G.words(MO, ids[2]), G.words(MO, ids[3])
    E = w13w.shape[0]
    x = G.as_f32(G.words(MO, ids[0]), dt).reshape(G.words(MO, ids[0]).shape)
    y = G.as_f32(G.words(MO, ids[1]), dt).reshape(G.words(MO, ids[1]).shape)
    w13 = G.as_f32(w13w, dt).reshape(w13w.shape)
    w2 = G.as_f32(w2w, dt).reshape(w2w.shape)
    return dict(name=NAMES[i], x=x, y=y, xw=G.words(MO, ids[0]), yw=G.words(MO, ids[1]), w13=w13, w2=w2,
                w13w=w13w, w2w=w2w, ids=topk, g=MO[p + "g"], emap=MO[p + "emap"] if has_map else None, act=act,
                rf=bool(rf), raw=raw, nl=nl, idx=idx, dt=dt, k=k, E=E, state=MO[p + "state"], cap=MO[p + "cap"],
                cap_x=MO[p + "cap_x"], cap_y=MO[p + "cap_y"], cap_ids=MO[p + "cap_ids"], cap_g=MO[p + "cap_g"])


def run_oracle(c, **over):
    H = c["x"].shape[1]
    cap = {"meta": np.zeros(4, np.int64), "x": np.zeros(H, np.float32), "y": np.zeros(H, np.float32),
           "ids": np.zeros(c["k"], np.int64), "g": np.zeros(c["k"], np.float32)}
    args = dict(x=c["x"], out=c["y"], topk_w=c["g"], topk_ids=c["ids"], w13=c["w13"], w2=c["w2"],
                expert_map=c["emap"], act=c["act"], routed_first=c["rf"], dtype=c["dt"], state=np.zeros(11, np.int64),
                cap=cap, raw=c["raw"], nlayers=c["nl"], index=c["idx"], line=6.0)
    args.update(over)
    return om.moe_check(**args)


def agrees(st, cap, c, z_tol=(0.3, 0.02)) -> list:
    """The differences between a state row / kept row and the reference's (empty: they agree)."""
    ref = c["state"]
    bad = []
    if list(st[om.C_CALLS:]) != list(ref[om.C_CALLS:]):
        bad.append(("counts", list(st[om.C_CALLS:]), list(ref[om.C_CALLS:])))
    z, zr = _f32(int(st[0]) >> 32), _f32(int(ref[0]) >> 32)
    if np.isinf(zr) or np.isinf(z):
        if not (np.isinf(z) and np.isinf(zr)):
            bad.append(("z", z, zr))
    elif abs(z - zr) > z_tol[0] + z_tol[1] * abs(zr):
        bad.append(("z", z, zr))
    if zr > 6:
        for col in (om.C_ROW, om.C_COL, om.C_OUT):
            if int(st[col]) & 0xFFFFFFFF != int(ref[col]) & 0xFFFFFFFF:
                bad.append((f"key {col}", int(st[col]) & 0xFFFFFFFF, int(ref[col]) & 0xFFFFFFFF))
    meta = [int(v) for v in cap["meta"]]
    if meta[:3] != [int(v) for v in c["cap"][:3]]:
        bad.append(("kept row", meta[:3], c["cap"][:3].tolist()))
    elif meta[0]:
        H = c["x"].shape[1]
        if not (np.array_equal(cap["x"][:H], c["cap_x"][:H]) and np.array_equal(cap["y"][:H], c["cap_y"][:H],
                                                                                 equal_nan=True)
                and np.array_equal(np.asarray(cap["ids"]), c["cap_ids"]) and np.allclose(cap["g"], c["cap_g"])):
            bad.append(("kept row values",))
    return bad


def test_fixture_inventory():
    assert len(NAMES) == 27 and sum(_f32(int(MO[f"c{i}_state"][0]) >> 32) > 6 for i in range(27)) == 4


@pytest.mark.parametrize("i", range(len(NAMES)))
def test_state_and_kept_row_match_reference(i):
    c = moe_case(i)
    st, cap, _ = run_oracle(c)
    bad = agrees(st, cap, c)
    assert not bad, (c["name"], bad)


def test_planted_mistake_fails(monkeypatch):
    """Dropping the routing weight from the recompute (planted in the oracle) makes clean rows score far off."""
    c = moe_case(NAMES.index("bf16_silu_clean"))
    real = om.recompute

    def no_weight(x_rows, ids, g, *a, **k):
        return real(x_rows, ids, np.ones_like(np.asarray(g, np.float32)), *a, **k)

    monkeypatch.setattr(om, "recompute", no_weight)
    st, cap, _ = run_oracle(c)
    assert agrees(st, cap, c)
