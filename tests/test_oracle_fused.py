"""The fused-check oracle (oracle/fused.py) against the reference's own answers (tests/golden/fused.npz, written by
tests/golden/make_golden.py from fused.py run in Triton's CPU interpreter).

  * zscores_from_stats on the reference's statistics: every checksum's score to 1e-3 relative (both sides float64
    sums of the same inputs; the fp32 norms are reduced in another order), verdicts and locations exactly;
  * block_stats of the exact product against the reference's statistics of its fp32 accumulator: within the
    reference's own tolerance 1e-5 (|C_block|_1 + |C_block|_2^2 + 1) (fused tests/_fused_compare.py);
  * checked_scores (the self-check's formula) with the exact product's statistics and the float64 expected side,
    against the reference's in-kernel fp32 scores: the reference's sums carry fp32 rounding that its clean scores
    show (at most 0.13 here), so scores agree to 0.3 + 2e-3 relative; Inf and unjudged exactly; verdicts and
    fault rows exactly;
  * block_sum_parts: the parts add up to the fp32 block sums (bf16: exactly; fp16: within 2^-38 of the block's
    largest possible sum, fused tests/test_fused.py:97-141), and the W-side norms are the frozen model's.
A planted mistake (the per-output noise terms dropped, in the oracle on the CPU) must fail the scores' check.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import fused as ofu
from tests import _golden as G
from tests.test_oracle_acc import flat_spans
from tests.test_oracle_golden import z_close

FU = G.load("fused.npz")
NAMES = G.names(FU)
LAYOUTS = ("plain", "w.t()", "gy.t()")


def fused_case(i):
    p = f"c{i}_"
    ids = [str(v) for v in FU[p + "ids"]]
    is16, lay, nfma, epoch, ir, ic, iv, kind = FU[p + "meta"]
    m, k, n = (int(v) for v in FU[p + "shape"])
    dt = "fp16" if is16 else "bf16"
    A = G.as_f32(G.words(FU, ids[0]), dt).reshape(m, k)
    B = G.as_f32(G.words(FU, ids[1]), dt).reshape(k, n)
    bias = G.as_f32(G.words(FU, ids[2]), dt).reshape(n) if ids[2] else None
    inject = None if ir < 0 else (int(ir), int(ic), float(iv))
    return dict(name=NAMES[i], A=A, B=B, bias=bias, dt=dt, layout=LAYOUTS[int(lay)], nfma=int(nfma) or None,
                epoch=int(epoch), inject=inject, kind=("fm", "zs", "chk")[int(kind)],
                stats=FU[p + "stats"] if p + "stats" in FU.files else None,
                zs=FU[p + "zs"] if p + "zs" in FU.files else None,
                result=FU[p + "result"] if p + "result" in FU.files else None,
                C=FU[p + "C"] if p + "C" in FU.files else None)


ZS = [i for i in range(len(NAMES)) if "_zs" in NAMES[i]]
FM = [i for i in range(len(NAMES)) if NAMES[i].endswith("_fm")]
CHK = [i for i in range(len(NAMES)) if "_chk" in NAMES[i]]


def exact_acc(c) -> np.ndarray:
    """The accumulator as exact arithmetic has it: A @ B + bias in float64, plus the injected fault."""
    C = c["A"].astype(np.float64) @ c["B"].astype(np.float64)
    if c["bias"] is not None:
        C = C + c["bias"].astype(np.float64)
    if c["inject"] is not None:
        r, col, v = c["inject"]
        C[r, col] += v
    return C


def test_fixture_inventory():
    assert len(ZS) == 2 * 7 * 5 + 1 and len(FM) == 14 and len(CHK) == 2 * 7 * 2 + 4


@pytest.mark.parametrize("i", ZS)
def test_zscores_from_stats_match_reference(i):
    c = fused_case(i)
    s = ofu.zscores_from_stats(c["A"], c["B"], c["stats"], c["bias"], nfma=c["nfma"], epoch=c["epoch"])
    ours = flat_spans(s.z, c["B"].shape[1])
    ok = z_close(ours, c["zs"])
    assert ok.all(), (c["name"], np.nonzero(~ok)[0][:5], ours[~ok][:5], c["zs"][~ok][:5])
    mz, row, blk, _ = c["result"]
    assert (s.max_z > 6) == (mz > 6) and (s.max_z < 0) == (mz < 0), (c["name"], s.max_z, mz)
    if mz > 6:
        assert (s.row, s.col_block) == (int(row), int(blk)), c["name"]


@pytest.mark.parametrize("i", FM)
def test_block_stats_of_exact_product_match_reference(i):
    c = fused_case(i)
    ours = ofu.block_stats(exact_acc(c), epoch=c["epoch"])
    ref = c["stats"]
    tol = 1e-5 * (np.abs(ours[..., 3:4]) + ours[..., 2:3] + 1)
    assert ours.shape == ref.shape
    assert (np.abs(ours - ref) <= tol).all(), (c["name"], np.abs(ours - ref).max())


def _checked(c, **kw):
    st = ofu.block_stats(exact_acc(c), epoch=c["epoch"])
    z, den, e = ofu.checked_scores(c["A"], c["B"], st, c["bias"], dtype=c["dt"], nfma=c["nfma"], epoch=c["epoch"],
                                   **kw)
    return flat_spans(z[None], c["B"].shape[1]), z, den, e


def close_chk(ours, ref):
    ours, ref = np.asarray(ours, np.float64), np.asarray(ref, np.float64)
    with np.errstate(invalid="ignore"):
        same_special = (np.isinf(ours) & np.isinf(ref)) | ((ours < 0) & (ref < 0))
        fin = np.isfinite(ours) & np.isfinite(ref) & (ours >= 0) & (ref >= 0)
        return same_special | (fin & (np.abs(ours - ref) <= 0.3 + 2e-3 * np.abs(ref)))


@pytest.mark.parametrize("i", CHK)
def test_checked_scores_match_reference(i):
    c = fused_case(i)
    ours, _, _, _ = _checked(c)
    ok = close_chk(ours, c["zs"])
    fin = np.isfinite(ours) & np.isfinite(c["zs"]) & (c["zs"] >= 0)
    print(f"{c['name']}: max |dz| {np.abs(ours[fin] - c['zs'][fin]).max():.3f}")
    assert ok.all(), (c["name"], np.nonzero(~ok)[0][:5], ours[~ok][:5], c["zs"][~ok][:5])
    mz, row, _, _ = c["result"]
    j = int(np.argmax(ours))
    oz = float(ours[j])
    assert (oz > 6) == (mz > 6) and (oz < 0 or (ours < 0).any() and oz <= 6) == (mz < 0), (c["name"], oz, mz)
    if mz > 6 and np.isfinite(mz):
        n = c["B"].shape[1]
        nbf = n // min(128, n)
        m = c["A"].shape[0]
        full = m * nbf * 2
        r = (j // 2) // nbf if j < full else (j - full) // 2
        assert r == int(row), (c["name"], r, row)


def test_planted_mistake_fails(monkeypatch):
    """A dropped term in the oracle (the per-output sqrt(k) and step terms of the noise, planted here on the CPU)
    moves the injected fault's score off the reference's."""
    i = next(i for i in CHK if NAMES[i].startswith("bf16_70x130x129") and NAMES[i].endswith("_chk_inj"))
    c = fused_case(i)
    good, _, _, _ = _checked(c)
    assert close_chk(good, c["zs"]).all()
    monkeypatch.setattr(ofu, "ACC_C2", 0.0)
    monkeypatch.setattr(ofu, "ACC_C3", 0.0)
    bad, _, _, _ = _checked(c)
    assert not close_chk(bad, c["zs"]).all()


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_block_sum_parts_are_exact_and_norms_are_the_model(dtype):
    rng = np.random.default_rng(0)
    K, N = 512, 200
    B = rng.standard_normal((K, N)).astype(np.float32) / 64
    if dtype == "fp16":
        B[: K // 2] *= 1e-3
        B = B.astype(np.float16).astype(np.float32)
    else:
        B = ofu._round16(B, "bf16")
    parts, scale, aux = ofu.block_sum_parts(B, dtype)
    for j in range(2):
        lo, hi = 128 * j, min(N, 128 * (j + 1))
        s = ofu._signs(hi - lo, 1, 0).astype(np.float64)
        bp = B[:, lo:hi].astype(np.float64).sum(1).astype(np.float32).astype(np.float64)
        bs = (B[:, lo:hi].astype(np.float64) * s).sum(1).astype(np.float32).astype(np.float64)
        got_p = parts[:, j, :3].astype(np.float64).sum(1) * scale[j]
        got_s = parts[:, j, 3:].astype(np.float64).sum(1) * scale[j]
        top = 128 * float(np.abs(B[:, lo:hi]).max())
        allowed = 0.0 if dtype == "bf16" else 2.0 ** -38 * top
        assert np.abs(got_p - bp).max() <= allowed and np.abs(got_s - bs).max() <= allowed, j
        assert abs(np.sqrt(aux[j, 1]) - np.linalg.norm(bp)) <= 1e-9 * np.linalg.norm(bp)
        assert abs(np.sqrt(aux[j, 0]) - np.linalg.norm(B[:, lo:hi].astype(np.float64))) <= 1e-9 * np.sqrt(aux[j, 0])
        if dtype == "fp16":
            assert 2 ** 14 <= top / scale[j] < 2 ** 15


def test_pow2_scale_matches_reference_rule():
    for wmax, want in ((1.0, 2.0 ** -7), (0.5, 2.0 ** -8), (float("inf"), 1.0), (1e-30, 2.0 ** -107), (1e-40, 2.0 ** -126), (700.0, 4.0)):
        assert ofu.pow2_scale(wmax) == want, (wmax, ofu.pow2_scale(wmax), want)
