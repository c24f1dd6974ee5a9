"""The quantized checks on the GPU (sdc_quant_check through sdcguard_amd.modes) against the reference's
modes.judge answers (tests/golden/quant.npz), the oracle (oracle/quant.py) on scaled fp8 problems, the
reference's +-127 known answer, and the 2048 x 7168 x 4096 int8 / fp8 workloads with injected faults."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant
from tests import _golden as G

pytestmark = pytest.mark.gpu

Q = G.load("quant.npz")
NCASES = sum(1 for k in Q.files if k.endswith("_nf"))


def _cases(mode):
    return [(i, f) for i in range(NCASES) if str(Q[f"q{i}_name"]).startswith(mode)
            for f in range(int(Q[f"q{i}_nf"]))]


def _case(i, f):
    a, b, c = Q[f"q{i}_a"], Q[f"q{i}_b"], Q[f"q{i}_c"].copy()
    r, j = (int(v) for v in Q[f"q{i}_f{f}_at"])
    c[r, j] = Q[f"q{i}_f{f}_v"]
    return str(Q[f"q{i}_name"]), a, b, c, Q[f"q{i}_f{f}_z"], int(Q[f"q{i}_f{f}_wrong"])


def _fp8(a_u8: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a_u8).cuda().view(torch.float8_e4m3fn)


@pytest.mark.parametrize("i,f", _cases("int8"))
def test_int8_matches_reference(i, f):
    from sdcguard_amd import modes
    name, a, b, c, z, wrong = _case(i, f)
    res = modes.judge("int8", torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), torch.from_numpy(c).cuda())
    assert res["wrong_blocks"] == wrong, name
    assert np.array_equal(np.isinf(res["z"].cpu().numpy()), np.isinf(z)), name


def _slack(A, B, sa, sb, C, W):
    """fp32 rounding of the expected side (MFMA accumulation of the three parts) in units of each block's noise."""
    Bs = B * sb[None, :]
    m, n = C.shape
    nb = -(-n // 128)
    out = np.zeros((m, nb))
    As = A * sa[:, None]
    for b in range(nb):
        lo, hi = 128 * b, min(n, 128 * b + 128)
        b2 = Bs[:, lo:hi] @ W[:, :hi - lo].T
        out[:, b] = (np.abs(As) @ np.abs(b2)).max(axis=1)
    return out * 2.0 ** -22


@pytest.mark.parametrize("i,f", _cases("fp8"))
def test_fp8_matches_reference(i, f):
    """Unit scales, fp32 result: modes.judge('fp8', nfma=16, unit=2^-14); z within 1e-3 (plus the expected side's
    fp32 rounding), verdicts and non-finite blocks identical."""
    from sdcguard_amd import modes
    name, a, b, c, z, wrong = _case(i, f)
    res = modes.judge("fp8", _fp8(a), _fp8(b), torch.from_numpy(c).cuda(), nfma=16, unit=modes.UNIT_FP8)
    zg = res["z"].cpu().numpy()
    assert res["wrong_blocks"] == wrong, (name, f)
    assert np.array_equal(np.isinf(zg), np.isinf(z)), name
    fin = np.isfinite(z)
    vals = quant.fp8_e4m3_values()
    A, B = vals[a], vals[b]
    sl = _slack(A, B, np.ones(A.shape[0]), np.ones(B.shape[1]), c, quant.patterns(1))
    den = 2.0 ** -14 * (np.sqrt((A ** 2).sum(1))[:, None] * 1.0 + 1.0)   # a lower bound of every block's noise
    tol = 1e-3 * np.maximum(1.0, np.abs(z)) + sl / den
    assert (np.abs(zg[fin] - z[fin]) <= tol[fin]).all(), (name, np.abs(zg[fin] - z[fin]).max())


def _scaled_problem(seed, m, k, n, out=torch.float32):
    """fp8 inputs with per-row / per-column scales 10^U(-3,-1) and C = sa_i sb_j (Aq @ Bq)_ij computed in float64
    on the GPU, rounded to `out`."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    Aq = (torch.randn(m, k, device="cuda", generator=g) * 4).clamp(-448, 448).to(torch.float8_e4m3fn)
    Bq = (torch.randn(k, n, device="cuda", generator=g) * 4).clamp(-448, 448).to(torch.float8_e4m3fn)
    sa = 10.0 ** (torch.rand(m, device="cuda", generator=g) * 2 - 3)
    sb = 10.0 ** (torch.rand(n, device="cuda", generator=g) * 2 - 3)
    C = ((Aq.double() @ Bq.double()) * sa.double()[:, None] * sb.double()[None, :]).to(out)
    return Aq, Bq, sa.float(), sb.float(), C


@pytest.mark.parametrize("shape", [(40, 256, 384), (7, 512, 300), (130, 1024, 1000)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_fp8_scaled_matches_oracle(shape, out):
    from sdcguard_amd import modes
    Aq, Bq, sa, sb, C = _scaled_problem(sum(shape), *shape, out=out)
    res = modes.judge("fp8", Aq, Bq, C, sa=sa, sb=sb)
    vals = quant.fp8_e4m3_values()
    A = vals[Aq.view(torch.uint8).cpu().numpy()]
    B = vals[Bq.view(torch.uint8).cpu().numpy()]
    o = quant.fp8_judge(A, B, sa.double().cpu().numpy(), sb.double().cpu().numpy(), C.double().cpu().numpy(),
                        quant.patterns(1), c_bf16=out == torch.bfloat16)
    zg = res["z"].cpu().numpy()
    assert res["wrong_blocks"] == o["wrong_blocks"] == 0
    assert np.allclose(zg, o["z"], rtol=1e-3, atol=2e-3), np.abs(zg - o["z"]).max()


@pytest.mark.parametrize("m,k,n", [(4096, 2048, 14336), (2048, 7168, 4096), (1000, 3072, 2048)])
@pytest.mark.parametrize("out", [torch.bfloat16, torch.float32])
def test_fp8_tall_gemm_matches_oracle(out, m, k, n):
    """The expected side on the tall-tile GEMM (fp8 A widened to bf16 in registers, the row norms in the same pass):
    128-row tiles over two depth halves where they fill the GPU (4096 x 2048 x 14336), else 64-row tiles over up to
    8 depth parts (2048 x 7168 x 4096: seven; 1000 x 3072 x 2048: six, a ragged last row tile).  Every block scores
    as the oracle scores it, and faults (a dequantized output 4 RMS off, a flipped exponent bit) are located."""
    from sdcguard_amd import modes
    Aq, Bq, sa, sb, C = _scaled_problem(71, m, k, n, out=out)
    consts = modes.QuantChecksums.make(Bq, sb)
    zs = torch.full((m, n // 128), -7.0, device="cuda")
    res = modes.resolve(modes.quant_zscores(Aq, consts, C, sa=sa, scores_out=zs))
    assert res["wrong_blocks"] == 0 and res["worst_z"] < 1.0, res
    vals = quant.fp8_e4m3_values()
    A = vals[Aq.view(torch.uint8).cpu().numpy()]
    B = vals[Bq.view(torch.uint8).cpu().numpy()]
    o = quant.fp8_judge(A, B, sa.double().cpu().numpy(), sb.double().cpu().numpy(), C.double().cpu().numpy(),
                        quant.patterns(1), c_bf16=out == torch.bfloat16)
    zg = zs.cpu().numpy()
    assert np.allclose(zg, o["z"], rtol=1e-3, atol=2e-3), np.abs(zg - o["z"]).max()
    print(f"fp8 {m}x{k}x{n} ({out}): max |dz| against the oracle {float(np.abs(zg - o['z']).max()):.2e}")
    rng = np.random.default_rng(9)
    for t in range(4):
        i, j = int(rng.integers(m)), int(rng.integers(n))
        c = C.clone()
        blk = c[i, (j // 128) * 128:(j // 128 + 1) * 128].float()
        if t % 2:
            c[i, j] = (c[i, j].float() + 4 * blk.pow(2).mean().sqrt()).to(out)
        elif out == torch.float32:
            v = c[i:i + 1, j].view(torch.int32)
            v ^= (1 << 30)
        else:
            v = c[i:i + 1, j].view(torch.int16)
            v ^= (1 << 14)
        zf = torch.full((m, n // 128), -7.0, device="cuda")
        res = modes.resolve(modes.quant_zscores(Aq, consts, c, sa=sa, scores_out=zf))
        of = quant.fp8_judge(A, B, sa.double().cpu().numpy(), sb.double().cpu().numpy(), c.double().cpu().numpy(),
                             quant.patterns(1), c_bf16=out == torch.bfloat16)
        # the faulty block scores as the oracle scores it, and the verdicts agree
        zfb, ofb = float(zf[i, j // 128]), float(of["z"][i, j // 128])
        assert (zfb == ofb) or abs(zfb - ofb) <= 1e-3 * max(1.0, abs(ofb)), (t, i, j, zfb, ofb)
        assert res["wrong_blocks"] == of["wrong_blocks"] and res["nonfinite_blocks"] == of.get(
            "nonfinite_blocks", res["nonfinite_blocks"]), (t, i, j, res, of["wrong_blocks"])
        if of["wrong_blocks"]:
            assert (res["row"], res["block"]) == (i, j // 128), (t, i, j, res)


def test_fp8_bf16_output_term_worst_case():
    """Outputs rounded to bf16 the same way by the most the format allows (tests/test_oracle_quant.py builds them):
    the HIP check scores every block as the oracle does -- 5.4 < z <= 5.66 for 2^-9 of the value, about 11 for 2^-8 --
    and flags the same blocks."""
    from sdcguard_amd import modes
    from tests.test_oracle_quant import worst_rounding_problem
    A, B, sa, sb, exact, c16 = worst_rounding_problem()
    Aq = torch.from_numpy(A).float().to(torch.float8_e4m3fn).cuda()
    Bq = torch.from_numpy(B).float().to(torch.float8_e4m3fn).cuda()
    consts = modes.QuantChecksums.make(Bq, torch.from_numpy(sb).float().cuda())
    C = torch.from_numpy(c16).bfloat16().cuda()
    zs = torch.full((C.shape[0], C.shape[1] // 128), -7.0, device="cuda")
    res = modes.resolve(modes.quant_zscores(Aq, consts, C, sa=torch.from_numpy(sa).float().cuda(), scores_out=zs))
    o = quant.fp8_judge(A, B, sa, sb, c16, quant.patterns(1), c_bf16=True)
    zg = zs.cpu().numpy()
    assert np.allclose(zg, o["z"], rtol=1e-3, atol=1e-3), (zg, o["z"])
    assert (5.4 < zg[:2]).all() and (zg[:2] <= np.sqrt(128) / 2 + 1e-3).all(), zg
    assert res["wrong_blocks"] == o["wrong_blocks"] == 2, res
    print(f"worst-case bf16 rounding: z {zg[:, 0]} (oracle {o['z'][:, 0]})")


def test_fp8_scaled_faults_located():
    from sdcguard_amd import modes
    Aq, Bq, sa, sb, C = _scaled_problem(9, 64, 512, 512)
    consts = modes.QuantChecksums.make(Bq, sb)
    for r, j, kind in [(3, 300, "add"), (0, 5, "nan"), (63, 130, "huge"), (10, 511, "inf")]:
        c = C.clone()
        blk = c[r, (j // 128) * 128:(j // 128 + 1) * 128]
        if kind == "add":
            c[r, j] += 0.5 * blk.pow(2).mean().sqrt()
        else:
            c[r, j] = {"nan": float("nan"), "huge": 1e30, "inf": float("inf")}[kind]
        res = modes.resolve(modes.quant_zscores(Aq, consts, c, sa=sa))
        assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (r, j // 128), (kind, res)


@pytest.mark.parametrize("m,k,n", [(1000, 3072, 2048), (64, 1024, 4096), (300, 2048, 1000)])
def test_int8_tall_gemm_matches_oracle(m, k, n):
    """An int8 check whose depth is a multiple of 1024 runs its expected side on the tall-tile GEMM (int8 MFMA on
    64-row tiles over up to 8 depth parts, one int32 plane per digit and part): every block's two exact sums equal
    the oracle's (1000 x 3072 x 2048: six parts, a ragged last row tile; 64 x 1024 x 4096: two; 300 x 2048 x 1000: a
    ragged last block), int8 values at both ends included, and a +1 in one output is that block alone."""
    from sdcguard_amd import modes
    g = torch.Generator(device="cuda").manual_seed(m + k + n)
    A = torch.randint(-128, 128, (m, k), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    B = torch.randint(-127, 128, (k, n), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    A[0, :] = -128
    A[1, :] = 127
    C = (A.double() @ B.double()).to(torch.int32)
    consts = modes.QuantChecksums.make(B)
    res = modes.resolve(modes.quant_zscores(A, consts, C))
    o = quant.int8_judge(A.cpu().numpy().astype(np.int64), B.cpu().numpy().astype(np.int64),
                         C.cpu().numpy().astype(np.int64), quant.patterns(1))
    assert res["wrong_blocks"] == o["wrong_blocks"] == 0, res
    i, j = m - 1, n - 1
    C[i, j] += 1
    zs = torch.full((m, -(-n // 128)), -7.0, device="cuda")
    res = modes.resolve(modes.quant_zscores(A, consts, C, scores_out=zs))
    assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (i, j // 128), res
    assert int((zs > 6).sum()) == 1 and float(zs[i, j // 128]) > 6


def test_int8_known_answer_at_the_largest_values():
    """Reference test_modes.py:47-64 on the GPU: +-127 everywhere at k = 1024, one output off by 1."""
    from sdcguard_amd import modes
    a = torch.full((64, 1024), 127, dtype=torch.int8, device="cuda")
    b = torch.full((1024, 256), 127, dtype=torch.int8, device="cuda")
    b[:, ::3] = -127
    c = (a.double() @ b.double()).to(torch.int32)
    assert int(c.abs().min()) == 16516096
    assert modes.judge("int8", a, b, c)["wrong_blocks"] == 0
    c[5, 200] += 1
    res = modes.judge("int8", a, b, c)
    assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (5, 1)


def test_int8_extreme_outputs_match_oracle():
    """The tile pass adds each int32 output as its two 16-bit halves: outputs at both ends of int32 (INT32_MIN,
    INT32_MAX, -1 in single outputs, and a block whose 128 outputs are all INT32_MAX) give exactly the oracle's
    per-block verdicts, which flag those blocks and no other."""
    from sdcguard_amd import modes
    m, k, n = 128, 1024, 512
    g = torch.Generator(device="cuda").manual_seed(31)
    A = torch.randint(-127, 128, (m, k), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    B = torch.randint(-127, 128, (k, n), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    C = (A.double() @ B.double()).to(torch.int32)
    j9 = 256 + int((C[9, 256:384] != -1).nonzero()[0])            # (an output of block 2 whose value is not -1)
    C[3, 5] = -2 ** 31
    C[7, 130] = 2 ** 31 - 1
    C[9, j9] = -1
    C[20, 384:512] = 2 ** 31 - 1
    consts = modes.QuantChecksums.make(B)
    zs = torch.full((m, n // 128), -7.0, device="cuda")
    res = modes.resolve(modes.quant_zscores(A, consts, C, scores_out=zs))
    o = quant.int8_judge(A.cpu().numpy().astype(np.int64), B.cpu().numpy().astype(np.int64),
                         C.cpu().numpy().astype(np.int64), quant.patterns(1))
    assert res["wrong_blocks"] == o["wrong_blocks"] == 4, (res, o["wrong_blocks"])
    flagged = (zs > 6).cpu().numpy()
    assert np.array_equal(flagged, o["bad"]), np.argwhere(flagged != o["bad"])
    assert {tuple(x) for x in np.argwhere(flagged)} == {(3, 0), (7, 1), (9, 2), (20, 3)}


def test_int8_2048x7168x4096_accumulator_bit_flips():
    """The quantized config at full size: A, B uniform on [-127, 127], C the exact int32 product; clean is exact;
    a flip of any one bit (0-30) of one int32 accumulator is exactly one wrong block, located; 8 trials."""
    from sdcguard_amd import modes
    g = torch.Generator(device="cuda").manual_seed(21)
    A = torch.randint(-127, 128, (2048, 7168), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    B = torch.randint(-127, 128, (7168, 4096), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    C = (A.double() @ B.double()).to(torch.int32)
    consts = modes.QuantChecksums.make(B)
    res = modes.resolve(modes.quant_zscores(A, consts, C))
    assert res["wrong_blocks"] == 0 and res["blocks"] == 2048 * 32
    rng = np.random.default_rng(5)
    for _ in range(8):
        i, j, bit = int(rng.integers(2048)), int(rng.integers(4096)), int(rng.integers(31))
        c = C.clone()
        c[i, j] ^= (1 << bit)
        res = modes.resolve(modes.quant_zscores(A, consts, c))
        assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (i, j // 128), (i, j, bit, res)


def test_fp8_2048x7168x4096_clean_and_faults():
    """The fp8 config at full size with log-uniform scales: clean (fp32 and bf16 outputs) raises nothing; a fault in
    the dequantized output of 4 typical outputs, or a flipped top exponent bit, is one wrong block, located."""
    from sdcguard_amd import modes
    Aq, Bq, sa, sb, C = _scaled_problem(33, 2048, 7168, 4096)
    consts = modes.QuantChecksums.make(Bq, sb)
    res = modes.resolve(modes.quant_zscores(Aq, consts, C, sa=sa))
    assert res["wrong_blocks"] == 0 and res["worst_z"] < 1.0, res
    res = modes.resolve(modes.quant_zscores(Aq, consts, C.bfloat16(), sa=sa))
    assert res["wrong_blocks"] == 0 and res["worst_z"] < 1.0, res
    rng = np.random.default_rng(6)
    for t in range(6):
        i, j = int(rng.integers(2048)), int(rng.integers(4096))
        c = C.clone()
        blk = c[i, (j // 128) * 128:(j // 128 + 1) * 128]
        if t % 2:
            c[i, j] += 4 * blk.pow(2).mean().sqrt()
        else:
            v = c[i:i + 1, j].view(torch.int32)
            v ^= (1 << 30)
        res = modes.resolve(modes.quant_zscores(Aq, consts, c, sa=sa))
        assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (i, j // 128), (t, i, j, res)


def test_int8_weights_at_minus_128():
    """int8 weights may hold -128: a block laid against the sign pattern (127 where it is +1, -128 where it is -1)
    has signed sums near 16384, whose high digit would be 128; the split keeps it at 127 and the check stays exact.
    The plain sum of a block of -128 entries, -16384, splits as (-128, 0)."""
    from sdcguard_amd import modes
    from sdcguard_amd.checksum import sign_table
    s = sign_table("cpu").view(128, 128)[127].to(torch.int32)              # the width-128 pattern
    g = torch.Generator(device="cuda").manual_seed(14)
    B = torch.randint(-127, 128, (512, 256), device="cuda", generator=g, dtype=torch.int32)
    B[:, 128:] = torch.where(s[None, :].cuda() > 0, torch.full_like(B[:, 128:], 127), -128)
    B[0, 128] = -127 if s[0] < 0 else 126                                  # 16383 at most in that block
    B = B.to(torch.int8)
    A = torch.randint(-127, 128, (64, 512), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    C = (A.double() @ B.double()).to(torch.int32)
    consts = modes.QuantChecksums.make(B)
    assert modes.resolve(modes.quant_zscores(A, consts, C))["wrong_blocks"] == 0
    c = C.clone()
    c[9, 200] += 1
    res = modes.resolve(modes.quant_zscores(A, consts, c))
    assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (9, 1)
    low = torch.full((128, 256), -128, dtype=torch.int8, device="cuda")
    A2 = A[:, :128].contiguous()
    C2 = (A2.double() @ low.double()).to(torch.int32)
    assert modes.resolve(modes.quant_zscores(A2, modes.QuantChecksums.make(low), C2))["wrong_blocks"] == 0


def test_int8_odd_depth_and_strided_operands():
    """Any depth and layout: k = 1001 (odd) and A a column slice starting at an odd byte (odd address, odd row
    stride 1003), which the C ABI copies into zero-padded buffers: clean is exact and matches the oracle's verdicts;
    one output off by one is one wrong block, located."""
    from sdcguard_amd import modes
    g = torch.Generator(device="cuda").manual_seed(31)
    m, k, n = 96, 1001, 384
    Abig = torch.randint(-127, 128, (m, k + 2), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    A = Abig[:, 1:1 + k]
    assert A.stride(0) % 2 == 1 and A.data_ptr() % 2 == 1
    B = torch.randint(-127, 128, (k, n), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    C = (A.double() @ B.double()).to(torch.int32)
    consts = modes.QuantChecksums.make(B)
    assert consts.parts.shape[-1] == k + 1
    assert modes.resolve(modes.quant_zscores(A, consts, C))["wrong_blocks"] == 0
    c = C.clone()
    c[17, 300] -= 1
    res = modes.resolve(modes.quant_zscores(A, consts, c))
    o = quant.int8_judge(A.cpu().numpy(), B.cpu().numpy(), c.cpu().numpy(), quant.patterns(1))
    assert res["wrong_blocks"] == o["wrong_blocks"] == 1 and (res["row"], res["block"]) == (17, 2), res


def test_fp8_any_depth_and_alignment():
    """fp8 A of depth 1000 (not a multiple of 32) read from a view 3 bytes off alignment (row stride 1003): the
    bounds-checked path scores as the oracle does, and a fault is located."""
    from sdcguard_amd import modes
    g = torch.Generator(device="cuda").manual_seed(32)
    m, k, n = 72, 1000, 260
    Abig = (torch.randn(m, k + 3, device="cuda", generator=g) * 4).to(torch.float8_e4m3fn)
    Aq = Abig[:, 3:3 + k]
    Bq = (torch.randn(k, n, device="cuda", generator=g) * 4).to(torch.float8_e4m3fn)
    sa = 10.0 ** (torch.rand(m, device="cuda", generator=g) * 2 - 3)
    sb = 10.0 ** (torch.rand(n, device="cuda", generator=g) * 2 - 3)
    C = ((Aq.double() @ Bq.double()) * sa.double()[:, None] * sb.double()[None, :]).float()
    res = modes.judge("fp8", Aq, Bq, C, sa=sa.float(), sb=sb.float())
    vals = quant.fp8_e4m3_values()
    o = quant.fp8_judge(vals[Aq.view(torch.uint8).cpu().numpy()], vals[Bq.view(torch.uint8).cpu().numpy()],
                        sa.cpu().numpy(), sb.cpu().numpy(), C.double().cpu().numpy(), quant.patterns(1))
    zg = res["z"].cpu().numpy()
    assert res["wrong_blocks"] == o["wrong_blocks"] == 0
    assert np.allclose(zg, o["z"], rtol=1e-3, atol=2e-3), np.abs(zg - o["z"]).max()
    c = C.clone()
    c[40, 259] = c[40, 259] * 1.5 + 1.0
    res = modes.judge("fp8", Aq, Bq, c, sa=sa.float(), sb=sb.float())
    assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (40, 2), res


def test_int8_row_block_check():
    """Row-block residuals of an int8 W8A8 GEMM (quant_rows_zscores: the column check of C^T = B^T A^T, B^T the
    layer's weight): clean is exact; the per-block verdicts equal the oracle's on the transposed operands; one wrong
    output is one wrong (column, row block), located, including in the narrower last row block."""
    from sdcguard_amd import modes
    g = torch.Generator(device="cuda").manual_seed(33)
    m, k, n = 300, 512, 256
    W = torch.randint(-127, 128, (n, k), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    A = torch.randint(-127, 128, (m, k), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    C = (A.double() @ W.double().t()).to(torch.int32)
    res = modes.judge_rows("int8", A, W.t(), C)
    assert res["wrong_blocks"] == 0 and res["blocks"] == n * 3
    for i, j in ((250, 77), (5, 255), (128, 0)):
        c = C.clone()
        c[i, j] += 3
        res = modes.judge_rows("int8", A, W.t(), c)
        o = quant.int8_judge(W.cpu().numpy(), A.t().cpu().numpy(), c.t().cpu().numpy(), quant.patterns(1))
        assert res["wrong_blocks"] == o["wrong_blocks"] == 1 and (res["row"], res["block"]) == (j, i // 128), res
        assert np.array_equal(np.isinf(res["z"].cpu().numpy()), o["bad"])


def test_fp8_row_block_check():
    """Row-block residuals of a scaled fp8 GEMM: per-(column, row block) z equal to the oracle's on the transposed
    operands (scales exchanged), clean raises nothing, a fault is located at its column and row block."""
    from sdcguard_amd import modes
    Aq, Bq, sa, sb, C = _scaled_problem(34, 200, 768, 384)
    res = modes.judge_rows("fp8", Aq, Bq, C, sa=sa, sb=sb)
    vals = quant.fp8_e4m3_values()
    A = vals[Aq.view(torch.uint8).cpu().numpy()]
    B = vals[Bq.view(torch.uint8).cpu().numpy()]
    o = quant.fp8_judge(B.T, A.T, sb.double().cpu().numpy(), sa.double().cpu().numpy(), C.double().cpu().numpy().T,
                        quant.patterns(1))
    zg = res["z"].cpu().numpy()
    assert res["wrong_blocks"] == o["wrong_blocks"] == 0
    assert np.allclose(zg, o["z"], rtol=1e-3, atol=2e-3), np.abs(zg - o["z"]).max()
    c = C.clone()
    col = c[:, 150]
    c[170, 150] += 4 * col[128:].pow(2).mean().sqrt()
    res = modes.judge_rows("fp8", Aq, Bq, c, sa=sa, sb=sb)
    assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (150, 1), res


def test_quant_row_checks_at_2048x7168x4096():
    """Both row-block checks at the quantized configuration's full size: int8 exact and clean, one flipped
    accumulator bit located; fp8 clean, one fault in the dequantized output located."""
    from sdcguard_amd import modes
    g = torch.Generator(device="cuda").manual_seed(35)
    A = torch.randint(-127, 128, (2048, 7168), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    W = torch.randint(-127, 128, (4096, 7168), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    C = (A.double() @ W.double().t()).to(torch.int32)
    assert modes.judge_rows("int8", A, W.t(), C)["wrong_blocks"] == 0
    c = C.clone()
    c[1000, 3000] ^= 1 << 9
    res = modes.judge_rows("int8", A, W.t(), c)
    assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (3000, 1000 // 128), res
    del A, W, C, c
    Aq, Bq, sa, sb, C = _scaled_problem(36, 2048, 7168, 4096)
    res = modes.judge_rows("fp8", Aq, Bq, C, sa=sa, sb=sb)
    assert res["wrong_blocks"] == 0 and res["worst_z"] < 1.0, res
    c = C.clone()
    c[77, 4000] += 4 * C[:128, 4000].pow(2).mean().sqrt()
    res = modes.judge_rows("fp8", Aq, Bq, c, sa=sa, sb=sb)
    assert res["wrong_blocks"] == 1 and (res["row"], res["block"]) == (4000, 0), res
