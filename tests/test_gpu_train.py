"""The training check (sdc_matmul_check through the C ABI: check_matmul / matmul_zscores / resolve) against the
reference's answers (tests/golden/train.npz), the oracle checksum by checksum, and the reference's own
invariant tests (tests/test_checksum.py of the reference: no false alarms on clean layers, zeroed 32-chunks,
NaN/Inf, top exponent-bit flips, the remainder block, bmm location, addmm with a 2-D bias and scaling, tiny
outputs), plus the 1024^3 bf16 workload with exponent-bit flips in half of 64 trials."""
from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import abft
from tests import _golden as G
from tests.test_oracle_golden import TRAIN, gemm_slack, train_case, z_close

pytestmark = pytest.mark.gpu


def _t(a: np.ndarray, dt: str) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16 if dt == "bf16" else
                                                                      torch.float16).cuda()


def _scores(A, B, C, bias=None, **kw):
    from sdcguard_amd.checksum import matmul_zscores, resolve
    bc = C.shape[0] if C.dim() == 3 else 1
    m, n = C.shape[-2], C.shape[-1]
    nb = -(-n // min(128, n))
    zs = torch.full((bc, m, nb, 2), -7.0, device="cuda")
    st = matmul_zscores(A, B, C, bias, scores_out=zs, **kw)
    res = resolve([st])[0]
    return zs.cpu().numpy(), res


@pytest.mark.parametrize("i", range(len(G.names(TRAIN))))
def test_training_kernel_matches_reference_and_oracle(i):
    name = G.names(TRAIN)[i]
    A, B, C, bias, alpha, beta, dt = train_case(i)
    zs, res = _scores(_t(A, dt), _t(B, dt), _t(C, dt), None if bias is None else _t(bias, dt), alpha=alpha, beta=beta)
    o = abft.zscores(A, B, C, bias, alpha=alpha, beta=beta, dtype=dt, seed=1)
    ok = z_close(zs.reshape(-1), o.z.reshape(-1), gemm_slack(o.csb, o.den).reshape(-1))
    assert ok.all(), (name, np.nonzero(~ok)[0][:5], zs.reshape(-1)[~ok][:5], o.z.reshape(-1)[~ok][:5])
    mz, b, r, blk, noise = TRAIN[f"c{i}_result"]
    assert (res.max_z > 6) == (mz > 6) and (res.max_z < 0) == (mz < 0), (name, res.max_z, mz)
    if mz > 6:
        assert (res.row, res.col_block) == (int(r), int(blk)), (name, res, (r, blk))
        if C.ndim == 3:
            assert res.batch == int(b)


def make_layer(T, din, dout, dtype=torch.bfloat16, outliers=False, seed=0):
    """tests/test_checksum.py:11-20 of the reference."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, din, generator=g)
    if outliers:
        ch = torch.randperm(din, generator=g)[: max(1, din // 256)]
        x[:, ch] *= 40
    W = torch.randn(dout, din, generator=g) / math.sqrt(din)
    b = torch.randn(dout, generator=g) * 0.02
    x, W, b = x.to(dtype).cuda(), W.to(dtype).cuda(), b.to(dtype).cuda()
    return x, W, b, F.linear(x, W, b)


SHAPES = [(256, 512, 1024), (512, 1024, 256), (128, 768, 3072), (64, 2048, 1000)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("outliers", [False, True])
def test_no_false_alarms_on_clean_layers(dtype, outliers):
    from sdcguard_amd.checksum import check_linear
    torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    for i, (T, din, dout) in enumerate(SHAPES):
        x, W, b, y = make_layer(T, din, dout, dtype, outliers, seed=i)
        res = check_linear(x, W, b, y)
        assert res is not None and res.ok, f"false alarm: shape {(T, din, dout)} z={res.max_z:.2f}"


def _rate(y0, x, W, b, corrupt, trials=60):
    from sdcguard_amd.checksum import check_linear
    caught = 0
    for t in range(trials):
        y = y0.clone()
        corrupt(y, random.Random(t))
        caught += not check_linear(x, W, b, y).ok
    return caught / trials


def test_catches_zeroed_warp_chunk():
    x, W, b, y0 = make_layer(256, 1024, 2048, outliers=True)

    def zero_chunk(y, rng):
        r, c = rng.randrange(y.shape[0]), rng.randrange(y.shape[1] // 32) * 32
        y[r, c:c + 32] = 0

    assert _rate(y0, x, W, b, zero_chunk) >= 0.9


def test_catches_nan_and_inf():
    from sdcguard_amd.checksum import check_linear
    x, W, b, y0 = make_layer(128, 512, 512)
    for bad in (float("nan"), float("inf")):
        y = y0.clone()
        y[3, 7] = bad
        res = check_linear(x, W, b, y)
        assert not res.ok and res.nonfinite and res.row == 3 and res.col_block == 0


def _flip(y, i, bit):
    v = y.view(-1)[i:i + 1].contiguous().view(torch.int16).clone()
    v ^= (1 << bit) if bit < 15 else -32768
    y.view(-1)[i] = v.view(y.dtype)[0]


def test_catches_top_exponent_bit_flip():
    x, W, b, y0 = make_layer(128, 512, 1024)
    assert _rate(y0, x, W, b, lambda y, rng: _flip(y, rng.randrange(y.numel()), 14)) == 1.0


def test_remainder_block_is_checked():
    from sdcguard_amd.checksum import check_linear
    x, W, b, y0 = make_layer(64, 256, 1000)
    y = y0.clone()
    y[5, 960:992] = 0
    res = check_linear(x, W, b, y)
    assert not res.ok and res.row == 5 and res.col_block == 7


def test_bmm_clean_and_corrupted():
    from sdcguard_amd.checksum import check_matmul
    g = torch.Generator().manual_seed(1)
    A = torch.randn(4, 64, 128, generator=g).bfloat16().cuda()
    B = (torch.randn(4, 128, 256, generator=g) / math.sqrt(128)).bfloat16().cuda()
    C = torch.bmm(A, B)
    assert check_matmul(A, B, C).ok
    C2 = C.clone()
    C2[2, 10, 32:64] = 0
    res = check_matmul(A, B, C2)
    assert not res.ok and res.batch == 2 and res.row == 10


def test_addmm_with_2d_bias_and_scaling():
    from sdcguard_amd.checksum import check_matmul
    g = torch.Generator().manual_seed(2)
    A = torch.randn(64, 128, generator=g).bfloat16().cuda()
    B = (torch.randn(128, 256, generator=g) / math.sqrt(128)).bfloat16().cuda()
    bias = torch.randn(64, 256, generator=g).bfloat16().cuda()
    C = torch.addmm(bias, A, B, beta=0.5, alpha=2.0)
    assert check_matmul(A, B, C, bias, alpha=2.0, beta=0.5).ok


def test_fp32_is_skipped():
    from sdcguard_amd.checksum import check_matmul
    A, B = torch.randn(8, 8).cuda(), torch.randn(8, 8).cuda()
    assert check_matmul(A, B, A @ B) is None


@pytest.mark.parametrize("scale", [1e-12, 1e-18, 1e-20, 1e-22, 1e-24, 1e-26, 1e-30, 1e-36])
def test_tiny_outputs_never_false_alarm(scale):
    from sdcguard_amd.checksum import check_matmul
    g = torch.Generator().manual_seed(0)
    W = (torch.randn(768, 768, generator=g) * 0.02).bfloat16()
    for i in range(4):
        dY = (torch.randn(256, 768, generator=g) * scale).bfloat16()
        dX = (dY.float() @ W.float()).bfloat16()
        res = check_matmul(dY.cuda(), W.cuda(), dX.cuda())
        assert res.ok, f"false alarm at scale {scale}: z={res.max_z}"


def test_strided_views_and_shared_b():
    """Transposed operands (a weight gradient's dY^T) and a bmm with one B shared by the batches."""
    from sdcguard_amd.checksum import check_matmul
    g = torch.Generator().manual_seed(5)
    dY = torch.randn(300, 96, generator=g).bfloat16().cuda()
    X = torch.randn(300, 200, generator=g).bfloat16().cuda()
    dW = dY.t() @ X
    zs, res = _scores(dY.t(), X, dW)
    o = abft.zscores(dY.t().float().cpu().numpy(), X.float().cpu().numpy(), dW.float().cpu().numpy(), seed=1)
    ok = z_close(zs.reshape(-1), o.z.reshape(-1), gemm_slack(o.csb, o.den).reshape(-1))
    assert ok.all() and res.ok
    A = torch.randn(3, 40, 64, generator=g).bfloat16().cuda()
    B = torch.randn(64, 130, generator=g).bfloat16().cuda()
    Bx = B.expand(3, 64, 130)
    C = torch.bmm(A, Bx)
    assert check_matmul(A, Bx, C).ok
    C[1, 7, 129] += 40
    r = check_matmul(A, Bx, C)
    assert not r.ok and (r.batch, r.row, r.col_block) == (1, 7, 1)


def test_bf16_1024_cubed_with_exponent_bit_flips():
    """1024^3 bf16, A and B ~ N(0,1), C = bf16(fp32 A @ B); 64 trials, trials 32-63 flip one random exponent bit
    (7-14) of one random element of C: the verdict of every trial matches the oracle's (outside |z - 6| < 0.3)."""
    from sdcguard_amd.checksum import check_matmul
    g = torch.Generator().manual_seed(1)
    A = torch.randn(1024, 1024, generator=g).bfloat16()
    B = torch.randn(1024, 1024, generator=g).bfloat16()
    C = (A.float() @ B.float()).bfloat16()
    Ad, Bd = A.cuda(), B.cuda()
    Af, Bf = A.float().numpy(), B.float().numpy()
    rng = np.random.default_rng(64)
    agree = band = 0
    for trial in range(64):
        Ct = C.clone()
        if trial >= 32:
            _flip(Ct, int(rng.integers(Ct.numel())), int(rng.integers(7, 15)))
        res = check_matmul(Ad, Bd, Ct.cuda())
        o = abft.zscores(Af, Bf, Ct.float().numpy(), seed=1)
        if abs(o.max_z - 6.0) < 0.3:
            band += 1
            continue
        assert res.ok == o.ok, (trial, res.max_z, o.max_z)
        if not o.ok:
            assert (res.row, res.col_block) == (o.row, o.col_block)
        agree += 1
    assert agree >= 62 and band <= 2


ROW_SHAPES = [(256, 512, 1024, torch.bfloat16), (300, 264, 1000, torch.bfloat16), (130, 1024, 520, torch.float16),
              (1, 96, 40, torch.bfloat16), (1100, 300, 37, torch.float16)]


@pytest.mark.parametrize("T,din,dout,dtype", ROW_SHAPES)
def test_transposed_weight_stage_matches_oracle(T, din, dout, dtype):
    """check_linear passes B = W.t() (k-contiguous rows): the column-read stage must give the oracle's scores,
    including k not a multiple of 8 or 256 and unaligned row strides."""
    x, W, b, y = make_layer(T, din, dout, dtype, outliers=True, seed=T)
    zs, res = _scores(x, W.t(), y, b)
    o = abft.zscores(x.float().cpu().numpy(), W.t().float().cpu().numpy(), y.float().cpu().numpy(),
                     b.float().cpu().numpy(), dtype="bf16" if dtype == torch.bfloat16 else "fp16", seed=1)
    ok = z_close(zs.reshape(-1), o.z.reshape(-1), gemm_slack(o.csb, o.den).reshape(-1))
    assert ok.all(), (np.nonzero(~ok)[0][:5], zs.reshape(-1)[~ok][:5], o.z.reshape(-1)[~ok][:5])
    assert res.ok and o.ok


@pytest.mark.parametrize("T,din,dout,dtype", ROW_SHAPES)
def test_row_block_check_matches_oracle(T, din, dout, dtype):
    """The row-block check (column-block check of y^T = W x^T + b[:, None]) against the oracle on the same
    transposed operands: per-checksum z, clean verdict; then a corrupted element is located at (column, row block)."""
    from sdcguard_amd.checksum import check_linear_rows, linear_rows_operands
    x, W, b, y = make_layer(T, din, dout, dtype, seed=T + 1)
    A, B, C, bias = linear_rows_operands(x, W, b, y)
    zs, res = _scores(A, B, C, bias)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    o = abft.zscores(A.float().cpu().numpy(), B.float().cpu().numpy(), C.float().cpu().numpy(),
                     bias.float().cpu().numpy(), dtype=dt, seed=1)
    ok = z_close(zs.reshape(-1), o.z.reshape(-1), gemm_slack(o.csb, o.den).reshape(-1))
    assert ok.all(), (np.nonzero(~ok)[0][:5], zs.reshape(-1)[~ok][:5], o.z.reshape(-1)[~ok][:5])
    assert res.ok and o.ok, (res.max_z, o.max_z)
    y2 = y.clone()
    r, c = T // 2, dout - 1
    y2[r, c] = y2[r, c] * 64 + 8
    res = check_linear_rows(x, W, b, y2)
    o = abft.check_matmul(*[t.float().cpu().numpy() for t in linear_rows_operands(x, W, b, y2)], dtype=dt, seed=1)
    assert not res.ok and not o.ok
    assert (res.row, res.col_block) == (c, r // 128) == (o.row, o.col_block)


def test_row_block_check_bit_flips_4096x4096x14336():
    """Full-size layer (x 4096x4096 N(0,1), W 14336x4096 N(0,0.02), y bf16): the row-block check is clean, and a
    flip of a top exponent bit of y[i, j] is located at (j, i // 128); one flip per trial, 8 trials."""
    from sdcguard_amd.checksum import check_linear_rows
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(4096, 4096, device="cuda", generator=g).bfloat16()
    W = (torch.randn(14336, 4096, device="cuda", generator=g) * 0.02).bfloat16()
    y = torch.nn.functional.linear(x, W)
    res = check_linear_rows(x, W, None, y)
    assert res.ok, res.max_z
    rng = random.Random(5)
    for _ in range(8):
        i, j = rng.randrange(4096), rng.randrange(14336)
        y2 = y.clone()
        _flip(y2, i * 14336 + j, 14)
        res = check_linear_rows(x, W, None, y2)
        assert not res.ok and (res.row, res.col_block) == (j, i // 128), (i, j, res)
