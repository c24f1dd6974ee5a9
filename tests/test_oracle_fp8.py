"""The FP8 quantization-check oracle (oracle/serve_fp8.py) against the reference's answers (tests/golden/fp8.npz:
serve_fp8.quant_check_torch's state rows, written by tests/golden/make_golden.py) and torch's FP8 conversion.

  * every fixture case: the state row after the case's calls, exactly (integers and float bits);
  * the E4M3 conversion: bit for bit with torch's float8_e4m3fn on every bf16 and fp16 value (clamped to +-448),
    random fp32 values, exact ties and the subnormal / normal boundary;
  * a mistake planted in the oracle (the second sample's row constant) fails the fixture cases that corrupt that
    row.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import serve_fp8 as of8
from tests import _golden as G

F8 = G.load("fp8.npz")
NAMES = G.names(F8)


def fp8_case(i):
    p = f"c{i}_"
    ids = [str(v) for v in F8[p + "ids"]]
    dtc, recipe, real, mult, m, k, mq = (int(v) for v in F8[p + "meta"])
    xw = G.words(F8, ids[0])
    if dtc == 4:
        x = np.ascontiguousarray(xw.astype(np.uint16)).view(np.float32).reshape(m, k)
        dt = "fp32"
    else:
        dt = "bf16" if dtc == 0 else "fp16"
        x = G.as_f32(xw, dt).reshape(m, k)
    xq = G.words(F8, ids[1]).astype(np.int16).astype(np.int8).view(np.uint8).reshape(mq, k)
    ub, sref = F8[p + "ub"], F8[p + "sref"]
    return dict(name=NAMES[i], x=x, xw=xw, dt=dt, dtc=dtc, xq=xq, xs=F8[p + "xs"], recipe=recipe,
                ub=ub if ub.size else None, sref=sref if sref.size else None, real=real, mult=mult,
                steps=[int(s) for s in F8[p + "steps"]], state=F8[p + "state"])


def run_oracle(c):
    st = np.zeros(8, np.int64)
    for s in c["steps"]:
        st = of8.quant_check(c["x"], c["xq"], c["xs"], c["recipe"], c["ub"], c["sref"], c["real"], s, c["mult"], st)
    return st


def test_fixture_inventory():
    assert len(NAMES) == 54
    assert any(F8[f"c{i}_state"][of8.C_OUTSIDE] for i in range(len(NAMES)))
    assert any(F8[f"c{i}_state"][of8.C_STATIC] for i in range(len(NAMES)))


@pytest.mark.parametrize("i", range(len(NAMES)))
def test_state_rows_match_reference(i):
    c = fp8_case(i)
    got = run_oracle(c)
    assert got.tolist() == c["state"].tolist(), (c["name"], got.tolist(), c["state"].tolist())


def _torch_e4m3(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_conversion_matches_torch_on_every_16_bit_value():
    w = np.arange(1 << 16, dtype=np.uint32)
    bf = (w << 16).view(np.float32)
    fp = w.astype(np.uint16).view(np.float16).astype(np.float32)
    for v in (bf, fp):
        v = np.where(np.isnan(v), v, np.clip(v, -448, 448)).astype(np.float32)
        assert np.array_equal(of8.to_e4m3(v), _torch_e4m3(v))


def test_conversion_matches_torch_on_fp32_values_and_ties():
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(200000) * np.exp2(rng.integers(-14, 9, 200000))).astype(np.float32)
    codes = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    fin = np.isfinite(vals)
    s = np.sort(np.unique(vals[fin]))
    ties = ((s[1:] + s[:-1]) / 2).astype(np.float32)                       # exact midpoints of neighbours
    edge = np.array([2.0 ** -6, np.nextafter(np.float32(2.0 ** -6), np.float32(0)), 2.0 ** -9, 2.0 ** -10,
                     1.5 * 2.0 ** -9, 448.0, -0.0, 0.0, np.nan, -np.nan], np.float32)
    for x in (v, ties, -ties, edge):
        x = np.where(np.isnan(x), x, np.clip(x, -448, 448)).astype(np.float32)
        assert np.array_equal(of8.to_e4m3(x), _torch_e4m3(x)), x[of8.to_e4m3(x) != _torch_e4m3(x)][:5]


def test_planted_mistake_fails(monkeypatch):
    i = NAMES.index("bf16_tensor_values_two_steps")
    c = fp8_case(i)
    assert run_oracle(c).tolist() == c["state"].tolist()
    monkeypatch.setattr(of8, "ROW_B", 104723)
    assert run_oracle(c).tolist() != c["state"].tolist()
