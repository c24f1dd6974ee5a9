"""The MoE grouped-GEMM check (sdc_grouped_check through checksum.grouped_zscores / check_grouped_mm) against the
oracle per group (each group is checked as check_matmul(a[start:end], b[g], out[start:end]), guard.py:102-143),
the other torch._grouped_mm layouts through per-group checks, and the 4096-token top-8 / 64-expert workload with
Zipf(1.1) expert loads and one corrupted expert tile."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import abft
from tests.test_oracle_golden import gemm_slack, z_close

pytestmark = pytest.mark.gpu


def _grouped(sizes, k, n, dtype=torch.bfloat16, seed=0, w_scale=None):
    g = torch.Generator().manual_seed(seed)
    T = sum(sizes)
    a = torch.randn(T, k, generator=g).to(dtype).cuda()
    b = (torch.randn(len(sizes), k, n, generator=g) * (w_scale or 1 / math.sqrt(k))).to(dtype).cuda()
    offs = torch.tensor(np.cumsum(sizes), dtype=torch.int32).cuda()
    out = torch.empty(T, n, dtype=dtype, device="cuda")
    s = 0
    for e, c in enumerate(sizes):
        if c:
            out[s:s + c] = (a[s:s + c].float() @ b[e].float()).to(dtype)
        s += c
    return a, b, out, offs


@pytest.mark.parametrize("sizes,k,n", [([0, 37, 130, 1, 200], 256, 300), ([513, 0, 0, 700], 512, 128),
                                       ([5] * 20, 96, 40),
                                       # more groups than a workgroup gathers in LDS (one-row groups)
                                       ([1] * 100 + [0, 300], 64, 40)])
def test_grouped_scores_match_oracle_per_group(sizes, k, n):
    from sdcguard_amd.checksum import grouped_zscores, resolve_grouped
    a, b, out, offs = _grouped(sizes, k, n, seed=len(sizes))
    nb = -(-n // min(128, n))
    zs = torch.full((sum(sizes), nb, 2), -7.0, device="cuda")
    res = resolve_grouped(grouped_zscores(a, b, out, offs, scores_out=zs))
    zs = zs.cpu().numpy()
    s, j = 0, 0
    for e, c in enumerate(sizes):
        if c:
            o = abft.zscores(a[s:s + c].float().cpu().numpy(), b[e].float().cpu().numpy(),
                             out[s:s + c].float().cpu().numpy(), seed=1)
            got = zs[s:s + c].reshape(-1)
            ok = z_close(got, o.z.reshape(-1), gemm_slack(o.csb, o.den).reshape(-1))
            assert ok.all(), (e, np.nonzero(~ok)[0][:5], got[~ok][:5], o.z.reshape(-1)[~ok][:5])
            assert res[j].ok == o.ok
            j += 1
        s += c
    assert j == len(res)


def test_grouped_fault_located_in_its_group():
    from sdcguard_amd.checksum import check_grouped_mm
    sizes = [64, 0, 300, 17, 129]
    a, b, out, offs = _grouped(sizes, 256, 384, seed=3)
    assert all(r.ok for r in check_grouped_mm(a, b, out, offs))
    bad = out.clone()
    bad[64 + 200, 130:140] += 4.0                # group 2 (the second non-empty group), local row 200, block 1
    res = check_grouped_mm(a, b, bad, offs)
    flags = [not r.ok for r in res]
    assert flags == [False, True, False, False]
    assert (res[1].row, res[1].col_block) == (200, 1)
    past = torch.cat([out, out[:3]])             # rows past offs[-1] belong to no group
    past[-2] = float("nan")
    a2 = torch.cat([a, a[:3]])
    assert all(r.ok for r in check_grouped_mm(a2, b, past, offs))


def test_other_grouped_layouts_match_per_group_checks():
    """3-D x 2-D (grouped along n), 2-D x 2-D (grouped along k, empty group = an all-zero output) and 3-D x 3-D run
    one check per group, as guard._grouped_checks splits them."""
    from sdcguard_amd.checksum import check_grouped_mm, check_matmul
    g = torch.Generator().manual_seed(4)
    A3 = torch.randn(3, 32, 64, generator=g).bfloat16().cuda()
    B2 = (torch.randn(64, 200, generator=g) / 8).bfloat16().cuda()
    offs_n = torch.tensor([50, 50, 200], dtype=torch.int32).cuda()
    out = torch.zeros(32, 200, dtype=torch.bfloat16, device="cuda")
    out[:, :50] = (A3[0].float() @ B2[:, :50].float()).bfloat16()
    out[:, 50:200] = (A3[2].float() @ B2[:, 50:].float()).bfloat16()
    res = check_grouped_mm(A3, B2, out, offs_n)
    assert len(res) == 2 and all(r.ok for r in res)
    A2 = torch.randn(16, 90, generator=g).bfloat16().cuda()
    Bk = torch.randn(90, 24, generator=g).bfloat16().cuda()
    offs_k = torch.tensor([40, 40, 90], dtype=torch.int32).cuda()
    outk = torch.stack([(A2[:, :40].float() @ Bk[:40].float()).bfloat16(), torch.zeros(16, 24).bfloat16().cuda(),
                        (A2[:, 40:].float() @ Bk[40:].float()).bfloat16()])
    res = check_grouped_mm(A2, Bk, outk, offs_k)
    assert len(res) == 3 and all(r.ok for r in res)
    outk[1, 3, 5] = 1.0                          # an empty group's output must be all zeros
    assert [r.ok for r in check_grouped_mm(A2, Bk, outk, offs_k)] == [True, False, True]
    Bb = torch.randn(3, 64, 40, generator=g).bfloat16().cuda()
    outb = torch.bmm(A3, Bb)
    assert check_grouped_mm(A3, Bb, outb, None)[0].ok == check_matmul(A3, Bb, outb).ok is True


def _zipf_counts(tokens, experts, topk, s, gen):
    p = torch.tensor([1.0 / (r + 1) ** s for r in range(experts)], dtype=torch.float64)
    picks = torch.multinomial(p.expand(tokens, experts), topk, replacement=False, generator=gen)
    return torch.bincount(picks.reshape(-1), minlength=experts).tolist()


def test_moe_4096_tokens_top8_64_experts():
    """4096 tokens x top-8 over 64 experts with Zipf(1.1) loads, K = 2048, N = 1408, bf16: clean raises nothing;
    one corrupted 128 x 128 tile of one expert's output flags that expert (and only it), at the tile's block;
    6 trials."""
    from sdcguard_amd.checksum import check_grouped_mm, grouped_zscores, resolve_grouped
    gen = torch.Generator().manual_seed(7)
    sizes = _zipf_counts(4096, 64, 8, 1.1, gen)
    assert sum(sizes) == 32768
    a, b, out, offs = _grouped(sizes, 2048, 1408, seed=8, w_scale=0.02)
    res = check_grouped_mm(a, b, out, offs)
    assert len(res) == sum(1 for c in sizes if c) and all(r.ok for r in res), max(r.max_z for r in res)
    starts = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    nonempty = [e for e, c in enumerate(sizes) if c]
    rng = np.random.default_rng(9)
    for _ in range(6):
        e = int(rng.choice([x for x in nonempty if sizes[x] >= 1]))
        r0 = int(starts[e]) + int(rng.integers(0, max(1, sizes[e] - 127))) if sizes[e] > 128 else int(starts[e])
        rows = min(128, sizes[e])
        blk = int(rng.integers(0, 11))
        bad = out.clone()
        bad[r0:r0 + rows, blk * 128:(blk + 1) * 128] = torch.randn(rows, 128, device="cuda").bfloat16()
        st = grouped_zscores(a, b, bad, offs)
        res = resolve_grouped(st)
        flagged = [nonempty[i] for i, r in enumerate(res) if not r.ok]
        assert flagged == [e], (e, flagged)
        r = res[nonempty.index(e)]
        assert r.col_block == blk and 0 <= r.row < sizes[e]


def test_offsets_out_of_order_and_past_the_rows_decode_consistently():
    """Offsets are read as the clamped running maximum (both kernels and the decoder): a decreasing entry is an empty
    group and an entry past the rows is the rows; the results match the per-group checks of those slices, and the
    epoch keyword reaches the device path."""
    from sdcguard_amd.checksum import check_grouped_mm, check_matmul, grouped_zscores, resolve_grouped
    a, b, out, _ = _grouped([40, 30, 50], 128, 136, seed=21)
    offs = torch.tensor([70, 40, 500], dtype=torch.int32, device="cuda")   # as ends: 70, 70 (empty), 120 (rows)
    res = resolve_grouped(grouped_zscores(a, b, out, offs))
    want = [check_matmul(a[0:70], b[0], out[0:70]), check_matmul(a[70:120], b[2], out[70:120])]
    assert [r.ok for r in res] == [w.ok for w in want]
    assert [round(r.max_z, 3) for r in res] == pytest.approx([round(w.max_z, 3) for w in want], abs=0.05)
    offs[0] = 0                                                              # the caller reuses its buffer
    torch.cuda.synchronize()
    r2 = check_grouped_mm(a, b, out, torch.tensor([40, 70, 120], device="cuda"), epoch=3)
    assert len(r2) == 3


@pytest.mark.parametrize("sizes,k,n,dtype,with_bias", [([0, 37, 130, 1, 200], 256, 300, torch.bfloat16, False),
                                                       ([513, 0, 0, 700], 512, 128, torch.float16, True),
                                                       ([5] * 20, 96, 40, torch.bfloat16, True)])
def test_serving_form_equals_the_per_call_check(sizes, k, n, dtype, with_bias):
    """GroupedChecksums (the experts' constants made once) and grouped_zscores(..., checksums=): the same result
    rows and every score as the call that makes the constants itself, clean and with a corrupted tile, over two
    calls in a row on one set of constants, with and without a shared bias (bias added to the outputs)."""
    from sdcguard_amd.checksum import GroupedChecksums, grouped_zscores, resolve_grouped
    a, b, out, offs = _grouped(sizes, k, n, dtype=dtype, seed=len(sizes) + 5)
    bias = None
    if with_bias:
        bias = (torch.randn(n, generator=torch.Generator().manual_seed(2)) * 0.3).to(dtype).cuda()
        out = (out.float() + bias.float()).to(dtype)
    cs = GroupedChecksums(b, bias)
    nb = -(-n // min(128, n))
    bad = out.clone()
    r0 = sizes[0] + min(sizes[1], 3) if sizes[0] == 0 else 3
    bad[r0, : min(n, 9)] += 2.0
    for y in (out, bad, out):
        z1 = torch.full((sum(sizes), nb, 2), -7.0, device="cuda")
        z2 = torch.full((sum(sizes), nb, 2), -7.0, device="cuda")
        s1 = grouped_zscores(a, b, y, offs, bias, scores_out=z1)
        s2 = grouped_zscores(a, None, y, offs, scores_out=z2, checksums=cs)
        torch.cuda.synchronize()
        assert torch.equal(s1.results, s2.results)
        assert torch.equal(z1, z2)
        r1, r2 = resolve_grouped(s1), resolve_grouped(s2)
        assert [(r.ok, r.row, r.col_block) for r in r1] == [(r.ok, r.row, r.col_block) for r in r2]
    assert not all(r.ok for r in resolve_grouped(grouped_zscores(a, None, bad, offs, checksums=cs)))
