"""The fused GEMM + precise check (sdc_fused_mm, sdc_fused_mm_checked, sdc_matmul_check_acc_stats through fused.py)
against the reference's answers (tests/golden/fused.npz), the oracle, exact arithmetic and the reference's own
fused tests (tests/_fused_compare.py, tests/test_fused.py).

Tolerances:
  * output: correctly rounded give or take the fp32 accumulation's rounding, |y - exact| <= half a step (1.0001) +
    k 2^-24 (|A| @ |B| + |bias|) (the reference's criterion; the reference's own output words, from another
    summation order, differ where that rounding crosses a step);
  * statistics: 1e-5 (|C_block|_1 + |C_block|_2^2 + 1) against the exact product and the reference's;
  * zscores_from_stats on the reference's statistics: 1e-3 relative (z_close), verdicts and locations exactly;
  * self-check: against the reference 0.3 + 2e-3 relative (both sides carry their own fp32 rounding, which the
    reference's clean scores show); against the oracle's formula given this kernel's own expected sides and
    statistics, 1e-3 relative; the expected side within the model's own term C1 sqrt(32) u |a| |sums|_2 + 4 u |e|
    of the float64 value; verdicts and fault locations exactly.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import fused as ofu
from tests.test_oracle_acc import flat_spans
from tests.test_oracle_fused import CHK, FM, NAMES, ZS, close_chk, exact_acc, fused_case
from tests.test_oracle_golden import z_close

pytestmark = pytest.mark.gpu


def _tdt(c):
    return torch.bfloat16 if c["dt"] == "bf16" else torch.float16


def _dev(c):
    """The case's operands on the GPU, in the layout the reference used (strides preserved)."""
    dt = _tdt(c)
    A = torch.from_numpy(c["A"]).to(dt)
    B = torch.from_numpy(c["B"]).to(dt)
    if c["layout"] == "w.t()":
        B = B.t().contiguous().t()
    elif c["layout"] == "gy.t()":
        A = A.t().contiguous().t()
    A, B = A.to("cuda"), B.to("cuda")
    bias = torch.from_numpy(c["bias"]).to(dt).cuda() if c["bias"] is not None else None
    return A, B, bias


def _ulp(x: np.ndarray, dt: str) -> np.ndarray:
    mant, emin = (7, -126) if dt == "bf16" else (10, -14)
    e = np.floor(np.log2(np.maximum(np.abs(x), 1e-300))).clip(emin)
    return np.exp2(e - mant)


def _words(y: torch.Tensor) -> np.ndarray:
    return y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _check_output(c, y: torch.Tensor):
    A, B = c["A"].astype(np.float64), c["B"].astype(np.float64)
    exact = exact_acc(c)
    half = 0.5 * _ulp(exact, c["dt"])
    acc_err = A.shape[1] * 2.0 ** -24 * (np.abs(A) @ np.abs(B) + (np.abs(c["bias"]) if c["bias"] is not None else 0))
    got = y.float().cpu().numpy().astype(np.float64)
    bad = ~(np.abs(got - exact) <= half * 1.0001 + acc_err)
    assert not bad.any(), (c["name"], np.argwhere(bad)[:5])


def _stats_close(ours: np.ndarray, ref: np.ndarray) -> bool:
    tol = 1e-5 * (np.abs(ref[..., 3:4]) + ref[..., 2:3] + 1)
    return bool((np.abs(ours - ref) <= tol).all())


@pytest.mark.parametrize("i", FM)
def test_fused_mm_output_and_statistics(i):
    from sdcguard_amd import fused
    c = fused_case(i)
    print(c["name"], flush=True)
    A, B, b = _dev(c)
    y, st = fused.fused_mm(A, B, b)
    _check_output(c, y)
    ours = st.cpu().numpy()
    assert _stats_close(ours, ofu.block_stats(exact_acc(c))), c["name"]
    assert _stats_close(ours, c["stats"]), c["name"]
    w = _words(y)
    diff = w != c["C"].reshape(w.shape)
    print(f"{c['name']}: {int(diff.sum())} of {diff.size} output words differ from the reference's (both within "
          f"the accumulation's rounding of the exact value)")


@pytest.mark.parametrize("i", ZS)
def test_zscores_from_stats_match_reference(i):
    from sdcguard_amd import checksum as cs
    from sdcguard_amd import fused
    c = fused_case(i)
    print(c["name"], flush=True)
    A, B, b = _dev(c)
    m, n = A.shape[0], B.shape[1]
    nb = -(-n // 128)
    zs = torch.full((m, nb, 2), -7.0, device="cuda")
    stats = torch.from_numpy(c["stats"]).cuda()
    st = fused.zscores_from_stats(A, B, stats, b, nfma=c["nfma"], epoch=c["epoch"], scores_out=zs)
    r = cs.resolve([st])[0]
    ours = flat_spans(zs.cpu().numpy()[None], n)
    ok = z_close(ours, c["zs"])
    assert ok.all(), (c["name"], np.nonzero(~ok)[0][:5], ours[~ok][:5], c["zs"][~ok][:5])
    mz, row, blk, _ = c["result"]
    assert (r.max_z > 6) == (mz > 6) and (r.max_z < 0) == (mz < 0), (c["name"], r, mz)
    if mz > 6:
        assert (r.row, r.col_block) == (int(row), int(blk)), (c["name"], r)
    if c["inject"] is not None:                    # the same fault in this kernel's accumulator
        _, st2 = fused.fused_mm(A, B, b, inject=c["inject"])
        r2 = cs.resolve([fused.zscores_from_stats(A, B, st2, b)])[0]
        assert not r2.ok and (r2.row, r2.col_block) == (int(row), int(blk)), (c["name"], r2)


@pytest.mark.parametrize("i", CHK)
def test_self_check_matches_reference_and_oracle(i):
    from sdcguard_amd import checksum as cs
    from sdcguard_amd import fused
    c = fused_case(i)
    print(c["name"], flush=True)
    A, B, b = _dev(c)
    m, n = A.shape[0], B.shape[1]
    nb = -(-n // 128)
    zs = torch.full((m, nb, 2), -7.0, device="cuda")
    ex = torch.full((m, nb, 2), float("nan"), dtype=torch.float64, device="cuda")
    y, st = fused.fused_mm_checked(A, B, b, inject=c["inject"], nfma=c["nfma"], epoch=c["epoch"], scores_out=zs,
                                   expected_out=ex)
    r = cs.resolve([st])[0]
    z = zs.cpu().numpy()
    ours = flat_spans(z[None], n)
    ok = close_chk(ours, c["zs"])
    fin = np.isfinite(ours) & np.isfinite(c["zs"]) & (c["zs"] >= 0)
    print(f"{c['name']}: max |dz| against the reference {np.abs(ours[fin] - c['zs'][fin]).max():.3f}")
    assert ok.all(), (c["name"], np.nonzero(~ok)[0][:5], ours[~ok][:5], c["zs"][~ok][:5])
    mz, row, _, _ = c["result"]
    assert (r.max_z > 6) == (mz > 6) and (r.max_z < 0) == (mz < 0), (c["name"], r, mz)
    if mz > 6 and math.isfinite(mz):
        assert r.row == int(row), (c["name"], r, row)
    # the same accumulator as fused_mm: identical output words, and the statistics the score used
    y0, st0 = fused.fused_mm(A, B, b, inject=c["inject"], epoch=c["epoch"])
    assert torch.equal(y, y0), c["name"]
    e = ex.cpu().numpy()
    oz, _, _ = ofu.checked_scores(c["A"], c["B"], st0.cpu().numpy(), c["bias"], dtype=c["dt"], nfma=c["nfma"],
                                  epoch=c["epoch"], expected=e)
    okf = z_close(z.reshape(-1), oz.reshape(-1))
    assert okf.all(), (c["name"], np.nonzero(~okf)[0][:5], z.reshape(-1)[~okf][:5], oz.reshape(-1)[~okf][:5])
    # the expected side: within the model's own term of its float64 value
    _, _, e64 = ofu.checked_scores(c["A"], c["B"], st0.cpu().numpy(), c["bias"], dtype=c["dt"], epoch=c["epoch"])
    if np.isfinite(c["A"]).all():
        _expected_within_model(c, e, e64)


def _expected_within_model(c, e, e64):
    parts, scale, aux = ofu.block_sum_parts(c["B"], c["dt"], epoch=c["epoch"])
    an = np.sqrt((c["A"].astype(np.float64) ** 2).sum(1))[:, None]
    u = 2.0 ** -24
    for q in range(2):
        allowed = an * np.sqrt(aux[:, 1 + q])[None, :] * 0.6 * math.sqrt(min(32, c["A"].shape[1])) * u \
            + 4 * u * np.abs(e64[..., q]) + 1e-30
        err = np.abs(e[..., q] - e64[..., q])
        assert (err <= allowed).all(), (c["name"], q, float((err / allowed).max()))


def test_sub_rounding_error_caught_and_epochs():
    """_fused_compare.py:88-110: a fault of 0.2% of a typical output (under half a bf16 step) is caught by the fused
    check and not by the ordinary check of the bf16 output; another epoch's pattern is clean, and statistics of one
    epoch do not pass under another's."""
    from sdcguard_amd import checksum as cs
    from sdcguard_amd import fused
    g = torch.Generator().manual_seed(99)
    A = torch.randn(32, 128, generator=g).bfloat16().cuda()
    B = (torch.randn(128, 256, generator=g) / 128 ** 0.5).bfloat16().t().contiguous().t().cuda()
    b = (torch.randn(256, generator=g) * 0.5).bfloat16().cuda()
    Cc, stc = fused.fused_mm(A, B, b)
    typical = Cc.float().abs().median().item()
    delta = 2e-3 * typical
    Cd, std = fused.fused_mm(A, B, b, inject=(7, 200, delta))
    rf = cs.resolve([fused.zscores_from_stats(A, B, std, b)])[0]
    ro = cs.check_matmul(A, B, Cd, b)
    print(f"sub-rounding fault {delta:.2e}: fused z {rf.max_z:.1f}, bf16 output z {ro.max_z:.2f}, "
          f"outputs changed {int((Cd != Cc).sum())}")
    assert not rf.ok and rf.row == 7 and rf.col_block == 1
    assert ro.ok
    _, stk = fused.fused_mm_checked(A, B, b, inject=(7, 200, delta))
    rk = cs.resolve([stk])[0]
    assert not rk.ok and rk.row == 7 and rk.col_block == 1, rk
    r_e = cs.resolve([fused.zscores_from_stats(A, B, fused.fused_mm(A, B, b, epoch=3)[1], b, epoch=3)])[0]
    r_x = cs.resolve([fused.zscores_from_stats(A, B, stc, b, epoch=3)])[0]
    assert r_e.ok and r_e.max_z < 1.0 and not r_x.ok
    r_k = cs.resolve([fused.fused_mm_checked(A, B, b, epoch=3)[1]])[0]
    assert r_k.ok and r_k.max_z < 1.0


def test_nonfinite_empty_and_bad_shapes():
    from sdcguard_amd import checksum as cs
    from sdcguard_amd import fused
    g = torch.Generator().manual_seed(7)
    A = torch.randn(64, 256, generator=g).bfloat16().cuda()
    B = (torch.randn(256, 256, generator=g) / 16).bfloat16().cuda()
    b = torch.randn(256, generator=g).bfloat16().cuda()
    for bad in (float("inf"), float("nan")):
        _, st = fused.fused_mm(A, B, b, inject=(0, 0, bad))
        assert not cs.resolve([fused.zscores_from_stats(A, B, st, b)])[0].ok
        _, st = fused.fused_mm_checked(A, B, b, inject=(5, 7, bad))
        r = cs.resolve([st])[0]
        assert not r.ok and r.judged, (bad, r)
    A2 = A.clone()
    A2[3, 4] = float("inf")
    r = cs.resolve([fused.fused_mm_checked(A2, B, b)[1]])[0]
    assert r.ok and not r.judged, r
    C, st = fused.fused_mm_checked(A[:, :0], B[:0], b)
    assert cs.resolve([st])[0].ok and torch.equal(C, b.expand(64, 256))
    C, st = fused.fused_mm(A[:, :0], B[:0], b)
    assert torch.equal(C, b.expand(64, 256))
    assert cs.resolve([fused.zscores_from_stats(A[:, :0], B[:0], st, b)])[0].ok
    C, st = fused.fused_mm(A[:0], B, b)
    assert C.shape == (0, 256) and st.shape == (0, 2, 4)
    with pytest.raises(ValueError, match="shape mismatch"):
        fused.fused_mm(A, torch.randn(9, 3, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="bias"):
        fused.fused_mm(A, B, torch.randn(4, device="cuda"))
    with pytest.raises(RuntimeError, match="GPU"):
        fused.fused_mm(A.cpu(), B.cpu())


@pytest.mark.parametrize("dt,m,k,n,layout", [("bf16", 700, 1000, 900, "gy.t()"), ("fp16", 520, 2048, 384, "plain"),
                                             ("bf16", 257, 4096, 1000, "w.t()")])
def test_larger_products_against_oracle(dt, m, k, n, layout):
    """Several row and column tiles, padded depths, transposed operands, many depth slices: scores against the
    oracle's formula and the expected side against its float64 value; a 1% fault in a corner found."""
    from sdcguard_amd import checksum as cs
    from sdcguard_amd import fused
    print(dt, m, k, n, layout, flush=True)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    g = torch.Generator().manual_seed(m + k + n)
    A = torch.randn(m, k, generator=g).to(tdt)
    B = (torch.randn(k, n, generator=g) / k ** 0.5).to(tdt)
    b = (torch.randn(n, generator=g) * 0.5).to(tdt)
    c = dict(name=f"{dt}_{m}x{k}x{n}", A=A.float().numpy(), B=B.float().numpy(), bias=b.float().numpy(), dt=dt,
             layout=layout, nfma=16, epoch=0, inject=None)
    Ad, Bd, bd = _dev(c)
    nb = -(-n // 128)
    zs = torch.zeros((m, nb, 2), device="cuda")
    ex = torch.zeros((m, nb, 2), dtype=torch.float64, device="cuda")
    y, st = fused.fused_mm_checked(Ad, Bd, bd, nfma=16, scores_out=zs, expected_out=ex)
    r = cs.resolve([st])[0]
    assert r.ok and 0 <= r.max_z < 1.0, r
    _check_output(c, y)
    y0, st0 = fused.fused_mm(Ad, Bd, bd)
    assert torch.equal(y, y0)
    s0 = st0.cpu().numpy()
    assert _stats_close(s0, ofu.block_stats(exact_acc(c)))
    e = ex.cpu().numpy()
    oz, _, e64 = ofu.checked_scores(c["A"], c["B"], s0, c["bias"], dtype=dt, nfma=16)
    oz2, _, _ = ofu.checked_scores(c["A"], c["B"], s0, c["bias"], dtype=dt, nfma=16, expected=e)
    okf = z_close(zs.cpu().numpy().reshape(-1), oz2.reshape(-1))
    assert okf.all(), np.nonzero(~okf)[0][:5]
    _expected_within_model(c, e, e64)
    # a fault of 20 times the corner block's noise (at k = 4096 that is about 5% of a typical output)
    inj = (m - 1, n - 1, 20.0 * float(ofu.checked_scores(c["A"], c["B"], s0, c["bias"], dtype=dt, nfma=16)[1][-1, -1]))
    zs1 = torch.zeros((m, nb, 2), device="cuda")
    _, st1 = fused.fused_mm_checked(Ad, Bd, bd, nfma=16, inject=inj, scores_out=zs1)
    r1 = cs.resolve([st1])[0]
    assert not r1.ok and (r1.row, r1.col_block) == (m - 1, (n - 1) // 128), r1
    c1 = dict(c, inject=inj)
    oz1, _, _ = ofu.checked_scores(c["A"], c["B"], ofu.block_stats(exact_acc(c1)), c["bias"], dtype=dt, nfma=16)
    assert close_chk(zs1.cpu().numpy()[-1, -1], oz1[-1, -1]).all(), (zs1[-1, -1], oz1[-1, -1])
    print(f"clean max z {r.max_z:.3f} (oracle {float(oz.max()):.3f}); fault z {r1.max_z:.1f} "
          f"(oracle {float(oz1[-1, -1].max()):.1f})")


def test_full_size_product_faults_found():
    """4096 x 4096 x 4096 bf16 linear layer (x @ w.T): clean, then 12 single faults of 5% of a typical output in
    random places (at this depth the model's noise is about 2e-3 of a typical output per block, so 1% stays under
    the line), each found at its row and block; the output against hipBLASLt's (within the two roundings)."""
    from sdcguard_amd import checksum as cs
    from sdcguard_amd import fused
    m = k = n = 4096
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(m, k, device="cuda", generator=g).bfloat16()
    w = (torch.randn(n, k, device="cuda", generator=g) / 64).bfloat16()
    b = torch.randn(n, device="cuda", generator=g).bfloat16()
    y, st = fused.fused_mm_checked(x, w.t(), b, nfma=16)
    r = cs.resolve([st])[0]
    ref = torch.nn.functional.linear(x, w, b)
    d = (y.float() - ref.float()).abs()
    tol = (ref.float().abs() * 2.0 ** -7 + 1e-3)
    print(f"clean max z {r.max_z:.3f}; output vs hipBLASLt: max |dy| {float(d.max()):.3g}, "
          f"{int((y != ref).sum())} words differ")
    assert r.ok and 0 <= r.max_z < 1.5, r
    assert bool((d <= tol).all())
    typical = float(y.float().abs().median())
    rng = np.random.default_rng(3)
    for _ in range(12):
        i, j = int(rng.integers(m)), int(rng.integers(n))
        _, st = fused.fused_mm_checked(x, w.t(), b, nfma=16, inject=(i, j, 0.05 * typical))
        r = cs.resolve([st])[0]
        assert not r.ok and (r.row, r.col_block) == (i, j // 128), (r, i, j)
    y2, st2 = fused.fused_mm(x, w.t(), b)
    r2 = cs.resolve([fused.zscores_from_stats(x, w.t(), st2, b, nfma=16)])[0]
    assert torch.equal(y, y2) and r2.ok, r2
