"""The precise check of an fp32 output (sdc_matmul_check_acc through the C ABI: matmul_zscores_acc /
check_matmul_acc / resolve) against the reference's answers (tests/golden/acc.npz), the oracle checksum by checksum
on larger products, the reference's own precise-mode tests (empty products, huge outputs that cancel in both
checksums, partially unjudged checks keeping a real alarm, zero and tiny outputs staying judged), and a
2048 x 4096 x 4096 bf16 product (fp32 output from the GPU's own GEMM) with single mantissa-bit flips.

Tolerance: both sides are float64 on the GPU and in the reference; the noise's fp32 norms are reduced in another
order, so scores agree to 1e-3 relative (1e-3 absolute near 0); inf and the unjudged -1 exactly; verdicts and fault
locations exactly.  Each test prints the largest relative |dz| it saw.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import acc as oacc
from tests import _golden as G
from tests.test_oracle_acc import ACC, acc_case, flat_spans
from tests.test_oracle_golden import z_close

pytestmark = pytest.mark.gpu


def _t16(a: np.ndarray, dt: str) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16 if dt == "bf16" else
                                                                      torch.float16).cuda()


def _t32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def _scores(A, B, C, bias=None, **kw):
    from sdcguard_amd.checksum import matmul_zscores_acc, resolve
    bc = C.shape[0] if C.dim() == 3 else 1
    m, n = C.shape[-2], C.shape[-1]
    nb = -(-n // min(128, n))
    zs = torch.full((bc, m, nb, 2), -7.0, device="cuda")
    st = matmul_zscores_acc(A, B, C, bias, scores_out=zs, **kw)
    return zs.cpu().numpy(), resolve([st])[0]


def _max_rel(ours, ref) -> float:
    ours, ref = np.asarray(ours, np.float64).reshape(-1), np.asarray(ref, np.float64).reshape(-1)
    fin = np.isfinite(ours) & np.isfinite(ref) & (ref > 0)
    return float(np.max(np.abs(ours[fin] - ref[fin]) / np.maximum(1.0, ref[fin]))) if fin.any() else 0.0


def fp32_product(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """The GPU's own fp32 product of 16-bit operands (hipBLASLt with an fp32 output where torch offers it)."""
    try:
        return torch.mm(A, B, out_dtype=torch.float32)
    except (RuntimeError, TypeError):
        return A.float() @ B.float()


@pytest.mark.parametrize("i", range(len(G.names(ACC))))
def test_precise_kernel_matches_reference(i):
    name = G.names(ACC)[i]
    A, B, C, bias, alpha, beta, dt, nfma, epoch = acc_case(i)
    zs, res = _scores(_t16(A, dt), _t16(B, dt), _t32(C), None if bias is None else _t16(bias, dt), alpha=alpha,
                      beta=beta, nfma=nfma, epoch=epoch)
    ours = flat_spans(zs, C.shape[-1])
    ref = ACC[f"c{i}_zs"]
    ok = z_close(ours, ref)
    print(f"{name}: max relative |dz| {_max_rel(ours, ref):.2e}")
    assert ok.all(), (name, np.nonzero(~ok)[0][:5], ours[~ok][:5], ref[~ok][:5])
    mz, b, r, blk, _ = ACC[f"c{i}_result"]
    assert (res.max_z > 6) == (mz > 6) and (res.max_z < 0) == (mz < 0), (name, res.max_z, mz)
    if mz > 6:
        assert math.isinf(res.max_z) == math.isinf(mz), name
        assert (res.row, res.col_block) == (int(r), int(blk)), (name, res, (r, blk))
        if C.ndim == 3:
            assert res.batch == int(b)


@pytest.mark.parametrize("dt,m,k,n,bias,batch,nfma", [
    ("bf16", 256, 1024, 1000, None, 0, None),
    ("fp16", 200, 768, 512, "vec", 0, 16),
    ("bf16", 64, 4096, 384, "mat", 0, 16),
    ("bf16", 48, 512, 300, None, 3, None),
])
def test_precise_kernel_matches_oracle(dt, m, k, n, bias, batch, nfma):
    g = torch.Generator(device="cuda").manual_seed(m + k + n)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    shapeA = (batch, m, k) if batch else (m, k)
    shapeB = (batch, k, n) if batch else (k, n)
    A = torch.randn(*shapeA, device="cuda", generator=g).to(tdt)
    B = (torch.randn(*shapeB, device="cuda", generator=g) * 0.05).to(tdt)
    C = torch.bmm(A.float(), B.float()) if batch else fp32_product(A, B)
    bt, kw = None, {}
    if bias == "vec":
        bt = (torch.randn(n, device="cuda", generator=g)).to(tdt)
        C = 0.5 * C + 1.5 * bt.float()
        kw = dict(alpha=0.5, beta=1.5)
    elif bias == "mat":
        bt = torch.randn(m, n, device="cuda", generator=g).to(tdt)
        C = C + bt.float()
    C[..., m // 2, n - 3] += 1.0               # (batched: in every batch)
    zs, res = _scores(A, B, C, bt, nfma=nfma, **kw)
    o = oacc.acc_zscores(A.float().cpu().numpy(), B.float().cpu().numpy(), C.cpu().numpy(),
                         None if bt is None else bt.float().cpu().numpy(), nfma=nfma, seed=1, **kw)
    ok = z_close(zs.reshape(-1), o.z.reshape(-1))
    print(f"{dt} {m}x{k}x{n} bias={bias} batch={batch}: max relative |dz| {_max_rel(zs, o.z):.2e}")
    assert ok.all(), (np.nonzero(~ok.reshape(-1))[0][:5], zs.reshape(-1)[~ok][:5], o.z.reshape(-1)[~ok][:5])
    assert (res.max_z > 6) == (o.max_z > 6)
    assert res.row == m // 2 and res.col_block == (n - 3) // 128


def test_empty_products_and_huge_cancelling_outputs():
    from sdcguard_amd.checksum import _signs, check_matmul_acc
    for m, k, n in ((0, 64, 256), (8, 64, 0), (8, 0, 256)):
        A, B = torch.randn(m, k, device="cuda").bfloat16(), torch.randn(k, n, device="cuda").bfloat16()
        assert check_matmul_acc(A, B, A.float() @ B.float()).ok
    torch.manual_seed(0)
    A, B = torch.randn(8, 64, device="cuda").bfloat16(), torch.randn(64, 256, device="cuda").bfloat16()
    s0 = _signs(128, "cpu", 0)
    j = next(j for j in range(1, 128) if s0[j] == s0[0])
    for big in (1e18, 1e6):
        C32 = A.float() @ B.float()
        C32[2, 0], C32[2, j] = big, -big
        r = check_matmul_acc(A, B, C32)
        assert not r.ok and r.row == 2 and r.col_block == 0, r


def _mixed(case, corrupt):
    """The reference's tests/test_numeric_completeness.py:_mixed: rows in several tiles and a partial last block."""
    a = torch.ones(70, 8, dtype=torch.bfloat16, device="cuda")
    b = torch.ones(8, 260, dtype=torch.bfloat16, device="cuda")
    if case == "row":
        a[0] = float("nan")
    elif case == "block":
        b[:, :128] = float("nan")
    elif case == "remainder":
        b[:, 256:] = float("nan")
    elif case == "batch":
        a, b = a.repeat(2, 1, 1), b.repeat(2, 1, 1)
        a[0] = float("nan")
    c = a.float() @ b.float()
    if corrupt:
        c.reshape(-1, c.shape[-1])[-1, 200] = 1000.0
    return a, b, c


@pytest.mark.parametrize("case", ["row", "block", "remainder", "batch"])
@pytest.mark.parametrize("corrupt", [False, True])
def test_partial_unjudged_keeps_a_real_alarm(case, corrupt):
    from sdcguard_amd.checksum import UNJUDGED, check_matmul_acc
    a, b, c = _mixed(case, corrupt)
    r = check_matmul_acc(a, b, c)
    if corrupt:
        assert not r.ok and r.max_z > 6, r
    else:
        assert r.ok and r.max_z == UNJUDGED, r


def test_zero_and_tiny_outputs_stay_judged():
    from sdcguard_amd.checksum import check_matmul_acc
    for scale in (0.0, 1e-24, 1.0):
        a = torch.full((3, 8), scale, dtype=torch.bfloat16, device="cuda")
        b = torch.ones(8, 260, dtype=torch.bfloat16, device="cuda")
        r = check_matmul_acc(a, b, a.float() @ b.float())
        assert r.ok and r.max_z >= 0, (scale, r)


def test_full_size_product_with_mantissa_bit_flips():
    """2048 x 4096 x 4096 bf16 with the GPU's fp32 output: clean, then one mantissa bit (bit 21: a relative change
    of 2^-2) flipped at 16 places, each found at its (row, block) with z over the line unless the output is too
    close to 0 for a quarter of it to stand out of the block's noise."""
    from sdcguard_amd.checksum import check_matmul_acc, matmul_zscores_acc, resolve
    m, k, n = 2048, 4096, 4096
    g = torch.Generator(device="cuda").manual_seed(3)
    A = torch.randn(m, k, device="cuda", generator=g).bfloat16()
    B = (torch.randn(k, n, device="cuda", generator=g) * 0.02).bfloat16()
    C = fp32_product(A, B)
    clean = check_matmul_acc(A, B, C, nfma=16)
    print(f"clean max z {clean.max_z:.3f}")
    assert clean.ok and 0 <= clean.max_z < 6, clean
    rng = np.random.default_rng(7)
    found = 0
    for _ in range(16):
        i, j = int(rng.integers(m)), int(rng.integers(n))
        bad = C.clone()
        w = bad.view(torch.int32)
        w[i, j] ^= (1 << 21)
        st = matmul_zscores_acc(A, B, bad, nfma=16)
        r = resolve([st])[0]
        if not r.ok:
            assert (r.row, r.col_block) == (i, j // 128), (r, i, j)
            found += 1
        else:
            # the flip moves the value by a quarter of itself: only outputs near 0 stay under the line
            assert abs(float(C[i, j])) * 0.25 < 12 * clean.noise, (i, j, float(C[i, j]), r)
    print(f"bit-21 flips found: {found} / 16")
    assert found >= 12
