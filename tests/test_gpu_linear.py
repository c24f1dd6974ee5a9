"""Both block checksums of a linear layer from one pass over y (sdc_linear_check, through the C ABI).

Every checksum's score is compared with the oracle's (the serving check for the column blocks, the training check
of y^T = W x^T + b[:, None] for the row blocks; tolerance of tests/test_oracle_golden.py) and with the two separate
entry points (sdc_check_static, sdc_matmul_check on the transposed views); counts exactly; the located fault
exactly.  At the full 4096 x 4096 x 14336 layer, single-bit flips of y: the verdicts of both checks agree with the
separate checks' on every flip outside the band |z - 6| < 0.3, and the band count is reported."""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle import abft, serve_check
from tests.test_oracle_golden import gemm_slack, z_close

pytestmark = pytest.mark.gpu


def make(m, k, n, with_bias, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", generator=g).bfloat16()
    W = (torch.randn(n, k, device="cuda", generator=g) * 0.02).bfloat16()
    b = (torch.randn(n, device="cuda", generator=g) * 0.1).bfloat16() if with_bias else None
    y = torch.nn.functional.linear(x.float(), W.float(), None if b is None else b.float()).bfloat16()
    return x, W, b, y


def fused(x, W, b, y, cs, concurrent=True):
    from sdcguard_amd.linear import check_linear_both
    m, n = y.shape
    mb, nb = -(-m // 128), -(-n // 128)
    zc = torch.full((m, nb, 2), -7.0, device="cuda")
    zr = torch.full((n, mb, 2), -7.0, device="cuda")
    st, rr = check_linear_both(x, W, b, y, cs, col_scores=zc, row_scores=zr, concurrent=concurrent)
    torch.cuda.synchronize()
    return zc.cpu().numpy(), zr.cpu().numpy(), st.cpu().numpy(), rr.cpu().numpy()


def separate(x, W, b, y, cs):
    from sdcguard_amd.checksum import linear_rows_operands, matmul_zscores
    from sdcguard_amd.serve import STATE_COLS, check_static_impl
    m, n = y.shape
    mb, nb = -(-m // 128), -(-n // 128)
    zc = torch.full((m, nb, 2), -7.0, device="cuda")
    zr = torch.full((1, n, mb, 2), -7.0, device="cuda")
    st = torch.zeros(1, STATE_COLS, dtype=torch.int64, device="cuda")
    check_static_impl(x, y, *cs.tensors(True), st, 0, 6.0, 1e-20, scores_out=zc)
    rr = torch.zeros(3, dtype=torch.int64, device="cuda")
    matmul_zscores(*linear_rows_operands(x, W, b, y), out=rr, scores_out=zr)
    torch.cuda.synchronize()
    return zc.cpu().numpy(), zr.cpu().numpy()[0], st.cpu().numpy()[0], rr.cpu().numpy()


def zmax(key) -> float:
    return float(np.array([int(key) >> 32], np.uint32).view(np.float32)[0])


SHAPES = [(512, 640, 1000, True), (300, 256, 136, False), (129, 1032, 264, True), (1024, 4096, 1408, True),
          (256, 4104, 512, False), (100, 1030, 264, True),        # (x rows not 16-byte aligned)
          # register-streamed GEMMs (depth a multiple of 512, 64 tiles or more): a ragged checksum-column count,
          # then a ragged last row block and a row check narrower than its 64-column tile
          (2048, 1024, 8200, True), (2000, 512, 8200, False),
          # its tall-tile variant (128-row tiles over two depth halves) for both GEMMs, ragged last row tile
          (3000, 512, 12800, True)]


@pytest.mark.parametrize("m,k,n,with_bias", SHAPES)
@pytest.mark.parametrize("concurrent", [True, False])
def test_both_checks_match_the_oracle_and_the_separate_checks(m, k, n, with_bias, concurrent):
    from sdcguard_amd.checksum import linear_rows_operands
    from sdcguard_amd.serve import LayerChecksums
    x, W, b, y = make(m, k, n, with_bias, seed=m + k + n)
    y[m // 3, n // 2] = y[m // 3, n // 2].float() * 64 + 8                 # one corrupted element
    cs = LayerChecksums(W, b, 128)
    zc, zr, st, rr = fused(x, W, b, y, cs, concurrent)
    zc2, zr2, st2, rr2 = separate(x, W, b, y, cs)
    # against the two separate entry points: the same scores (only the order of fp32 additions differs)
    assert z_close(zc.reshape(-1), zc2.reshape(-1)).all()
    assert z_close(zr.reshape(-1), zr2.reshape(-1)).all()
    assert st[2] == 1 and st[3] == st2[3] and rr[2] == rr2[2]
    # against the oracle
    f = lambda t: t.float().cpu().numpy()                                    # noqa: E731
    c = serve_check.layer_constants(f(W), None if b is None else f(b), 128, "bf16", seed=1)
    o = serve_check.check_static(f(x), f(y), c, dtype="bf16", seed=1)
    ok = z_close(zc.reshape(-1), o.z.reshape(-1), gemm_slack(o.csb, o.den).reshape(-1))
    assert ok.all(), (np.nonzero(~ok)[0][:5], zc.reshape(-1)[~ok][:5], o.z.reshape(-1)[~ok][:5])
    A, B, C, bias = linear_rows_operands(x, W, b, y)
    orow = abft.zscores(f(A), f(B), f(C), None if bias is None else f(bias), dtype="bf16", seed=1)
    ok = z_close(zr.reshape(-1), orow.z.reshape(-1), gemm_slack(orow.csb, orow.den).reshape(-1))
    assert ok.all(), (np.nonzero(~ok)[0][:5], zr.reshape(-1)[~ok][:5], orow.z.reshape(-1)[~ok][:5])
    # the fault, located by both checks as the separate checks and the oracle locate it
    fc, fr = int(st[0]) & 0xFFFFFFFF, int(rr[0]) & 0xFFFFFFFF
    nb, mb = -(-n // 128), -(-m // 128)
    assert zmax(st[0]) > 6 and (fc // 2) == (m // 3) * nb + (n // 2) // 128
    assert zmax(rr[0]) > 6 and (fr // 2) == (n // 2) * mb + (m // 3) // 128
    assert (fc // 2, fr // 2) == ((int(st2[0]) & 0xFFFFFFFF) // 2, (int(rr2[0]) & 0xFFFFFFFF) // 2)
    dz = max(float(np.nanmax(np.abs(np.where(np.isfinite(zc2), zc - zc2, 0)))),
             float(np.nanmax(np.abs(np.where(np.isfinite(zr2), zr - zr2, 0)))))
    print(f"{m}x{k}x{n}: max |dz| against the separate checks {dz:.2e}")


def _flip(y: torch.Tensor, flat: int, bit: int) -> None:
    v = y.view(-1)[flat:flat + 1].view(torch.int16)
    y.view(-1)[flat] = (v ^ (1 << bit)).view(torch.bfloat16)[0]


def test_full_size_layer_single_bit_flips():
    """x 4096x4096 N(0,1), W 14336x4096 N(0,0.02), y = x W^T in bf16: every clean score of both checks against the
    oracle (the serving check on y, the training check on y^T = W x^T); then 16 trials each flipping one random bit
    (exponent or mantissa) of one random element of y: the flipped row's column-block scores and the flipped column's
    row-block scores against the oracle's for that row and column, every other score as clean, and the verdicts
    against the separate checks' outside the band |z - 6| < 0.3; a flagged flip is located at the same place.
    Prints the largest |dz| against the oracle and the band count."""
    from sdcguard_amd.checksum import linear_rows_operands
    from sdcguard_amd.serve import LayerChecksums
    x, W, b, y = make(4096, 4096, 14336, False, seed=3)
    cs = LayerChecksums(W, None, 128)
    zc, zr, st, rr = fused(x, W, None, y, cs)
    assert zmax(st[0]) < 6 and zmax(rr[0]) < 6, (zmax(st[0]), zmax(rr[0]))
    f = lambda t: t.float().cpu().numpy()                                    # noqa: E731
    xf, Wf, yf = f(x), f(W), f(y)
    c = serve_check.layer_constants(Wf, None, 128, "bf16", seed=1)
    o = serve_check.check_static(xf, yf, c, dtype="bf16", seed=1)
    ok = z_close(zc.reshape(-1), o.z.reshape(-1), gemm_slack(o.csb, o.den).reshape(-1))
    assert ok.all(), (np.nonzero(~ok)[0][:5], zc.reshape(-1)[~ok][:5], o.z.reshape(-1)[~ok][:5])
    xt = np.ascontiguousarray(xf.T)
    orow = abft.zscores(Wf, xt, np.ascontiguousarray(yf.T), None, dtype="bf16", seed=1)
    ok = z_close(zr.reshape(-1), orow.z.reshape(-1), gemm_slack(orow.csb, orow.den).reshape(-1))
    assert ok.all(), (np.nonzero(~ok)[0][:5], zr.reshape(-1)[~ok][:5], orow.z.reshape(-1)[~ok][:5])
    dz_clean = max(float(np.abs(zc - o.z.reshape(zc.shape)).max()), float(np.abs(zr - orow.z.reshape(zr.shape)).max()))
    rng = random.Random(11)
    band = agree = flagged = 0
    worst_dz = 0.0
    for trial in range(16):
        i, j, bit = rng.randrange(4096), rng.randrange(14336), rng.randrange(0, 15)
        y2 = y.clone()
        _flip(y2, i * 14336 + j, bit)
        zc2, zr2, st2, rr2 = fused(x, W, None, y2, cs)
        zs, zrs, sts, rrs = separate(x, W, None, y2, cs)
        # every other row / column scores as clean
        keep_r = np.ones(4096, bool)
        keep_r[i] = False
        keep_c = np.ones(14336, bool)
        keep_c[j] = False
        assert np.array_equal(zc2[keep_r], zc[keep_r]) and np.array_equal(zr2[keep_c], zr[keep_c]), trial
        # the flipped row and column against the oracle
        y2f = y2[i:i + 1].float().cpu().numpy()
        orr = serve_check.check_static(xf[i:i + 1], y2f, c, dtype="bf16", seed=1)
        okr = z_close(zc2[i].reshape(-1), orr.z.reshape(-1), gemm_slack(orr.csb, orr.den).reshape(-1))
        assert okr.all(), (trial, bit, zc2[i].reshape(-1)[~okr][:4], orr.z.reshape(-1)[~okr][:4])
        ycol = y2[:, j:j + 1].float().cpu().numpy().T
        occ = abft.zscores(Wf[j:j + 1], xt, np.ascontiguousarray(ycol), None, dtype="bf16", seed=1)
        okc = z_close(zr2[j].reshape(-1), occ.z.reshape(-1), gemm_slack(occ.csb, occ.den).reshape(-1))
        assert okc.all(), (trial, bit, zr2[j].reshape(-1)[~okc][:4], occ.z.reshape(-1)[~okc][:4])
        fin_r, fin_c = np.isfinite(orr.z), np.isfinite(occ.z)
        worst_dz = max(worst_dz, float(np.abs(zc2[i].reshape(-1) - orr.z.reshape(-1))[fin_r.reshape(-1)].max()),
                       float(np.abs(zr2[j].reshape(-1) - occ.z.reshape(-1))[fin_c.reshape(-1)].max()))
        for got, want, loc in ((st2, sts, (i * 112 + j // 128)), (rr2, rrs, (j * 32 + i // 128))):
            zg, zw = zmax(got[0]), zmax(want[0])
            if abs(zw - 6.0) < 0.3 or abs(zg - 6.0) < 0.3:
                band += 1
                continue
            assert (zg > 6) == (zw > 6), (trial, bit, zg, zw)
            agree += 1
            if zg > 6:
                flagged += 1
                assert (int(got[0]) & 0xFFFFFFFF) // 2 == loc, (trial, bit)
    print(f"clean: max |dz| against the oracle {dz_clean:.2e}; 16 single-bit flips x 2 checks: {agree} verdicts "
          f"agree, {band} in the band, {flagged} flagged; max |dz| of the flipped row and column against the oracle "
          f"{worst_dz:.2e}")
    assert band <= 2


@pytest.mark.parametrize("m,k,n,with_bias", [(512, 512, 1024, True), (3000, 512, 12800, False)])
def test_non_finite_and_impossible_outputs(m, k, n, with_bias):
    """NaN, +Inf, -Inf and a huge finite value (an "impossible" checksum) in y: every score of both checks equals the
    separate checks' and the oracle's (special scores exactly), so the y pass's full non-finite rules agree with the
    fast scoring of clean pairs beside them; the unjudged counts match."""
    from sdcguard_amd.checksum import linear_rows_operands
    from sdcguard_amd.serve import LayerChecksums
    x, W, b, y = make(m, k, n, with_bias, seed=m + n + 7)
    y[3, 5] = float("nan")
    y[m // 2, n - 3] = float("inf")
    y[m - 1, n // 3] = float("-inf")
    y[m // 4, n // 5] = 1e30
    cs = LayerChecksums(W, b, 128)
    zc, zr, st, rr = fused(x, W, b, y, cs)
    zc2, zr2, st2, rr2 = separate(x, W, b, y, cs)
    assert z_close(zc.reshape(-1), zc2.reshape(-1)).all()
    assert z_close(zr.reshape(-1), zr2.reshape(-1)).all()
    assert st[3] == st2[3] and rr[2] == rr2[2]
    f = lambda t: t.float().cpu().numpy()                                    # noqa: E731
    c = serve_check.layer_constants(f(W), None if b is None else f(b), 128, "bf16", seed=1)
    o = serve_check.check_static(f(x), f(y), c, dtype="bf16", seed=1)
    assert z_close(zc.reshape(-1), o.z.reshape(-1), gemm_slack(o.csb, o.den).reshape(-1)).all()
    A, B, C, bias = linear_rows_operands(x, W, b, y)
    orow = abft.zscores(f(A), f(B), f(C), None if bias is None else f(bias), dtype="bf16", seed=1)
    assert z_close(zr.reshape(-1), orow.z.reshape(-1), gemm_slack(orow.csb, orow.den).reshape(-1)).all()
    nb = -(-n // 128)
    assert np.isinf(zc[m // 4, (n // 5) // 128]).any() and np.isinf(zc[m // 2, (n - 3) // 128]).any()
    assert zmax(st[0]) > 6 and zmax(rr[0]) > 6 and nb > 0
