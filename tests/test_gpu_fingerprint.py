"""Fingerprint kernels on the GPU: bit-exact against the oracle (numpy uint64 and brute-force Python ints) on the
reference's own probe cases (_fingerprint._probe_ok, serve_weights.verify_kernel) and its known-pattern tests."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fingerprint as F

pytestmark = pytest.mark.gpu


def _np(t: torch.Tensor) -> np.ndarray:
    """Raw values as numpy (bf16 as its int16 words: numpy has no bf16)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.numpy()


def test_fp3_probe_cases_of_the_reference():
    """_fingerprint.py:79-94's probe tensors (seed 251): int16/int8 views, sizes that are not a multiple of the
    kernel's block, saturated words."""
    from sdcguard_amd.recompute import fingerprint_bits
    g = torch.Generator(device="cpu").manual_seed(251)
    cases = [torch.randint(-32768, 32768, (3 * 4096 + 19,), generator=g, dtype=torch.int32).to(torch.int16),
             torch.randint(-128, 128, (4096 + 3,), generator=g, dtype=torch.int32).to(torch.int8),
             torch.randint(-32768, 32768, (250,), generator=g, dtype=torch.int32).to(torch.int16),
             torch.full((2259,), 32767, dtype=torch.int16), torch.full((4096,), -32768, dtype=torch.int16)]
    for c in cases:
        got = _np(fingerprint_bits(c.cuda()))
        assert np.array_equal(got, F.fp3(_np(c))), (c.dtype, c.numel())
        if c.numel() < 3000:
            assert tuple(got) == F.fp3_py(_np(c))


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16, torch.float64, torch.uint8, torch.bool])
def test_fp3_of_tensors(dt):
    from sdcguard_amd.recompute import fingerprint
    g = torch.Generator().manual_seed(0)
    for n in (1, 7, 4095, 4096 * 3 + 5, 1 << 20 | 3):
        if dt in (torch.uint8, torch.bool):
            t = torch.randint(0, 2 if dt == torch.bool else 256, (n,), generator=g).to(dt)
        else:
            t = (torch.randn(n, generator=g) * 100).to(dt)
        got = _np(fingerprint(t.cuda()))
        assert np.array_equal(got, F.fp3(F.fp3_words(_np(t)))), (dt, n)


def test_fp3_unaligned_view():
    from sdcguard_amd.recompute import fingerprint_bits
    base = torch.randint(-32768, 32768, (10001,), dtype=torch.int32).to(torch.int16).cuda()
    v = base[3:]                                      # 6-byte offset: the element-wise kernel
    assert np.array_equal(_np(fingerprint_bits(v)), F.fp3(_np(v)))


def test_fp3_known_patterns_of_the_reference():
    """test_recompute.py:247-290: +1/-2/+1 neighbours, a swap of 1.0 and 0.99609381 597 apart, an fp64 word
    change: each must change the fingerprint (on the GPU, as the oracle computes it)."""
    from sdcguard_amd.recompute import fingerprint
    x = torch.randn(1000, generator=torch.Generator().manual_seed(0)).bfloat16()
    y = x.clone()
    r = y.view(torch.int16)
    r[10] += 1
    r[11] -= 2
    r[12] += 1
    fx, fy = _np(fingerprint(x.cuda())), _np(fingerprint(y.cuda()))
    assert not np.array_equal(fx, fy) and np.array_equal(fx, F.fp3(F.fp3_words(_np(x))))
    x = torch.zeros(1000)
    x.view(torch.int32)[3] = 0x3F800000
    x.view(torch.int32)[600] = 0x3F7F0001
    y = x.clone()
    y[3], y[600] = x[600], x[3]
    assert not np.array_equal(_np(fingerprint(x.cuda())), _np(fingerprint(y.cuda())))
    x = torch.ones(100, dtype=torch.float64)
    x.view(torch.int64)[5] = 0x3FF0000000020000
    y = x.clone()
    y.view(torch.int64)[5] = 0x3FF0000100000001
    assert not np.array_equal(_np(fingerprint(x.cuda())), _np(fingerprint(y.cuda())))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float64, torch.uint8])
def test_fp2_verify_kernel_cases_of_the_reference(dt):
    """serve_weights.py:251-290's cases: n in (1, 7, 4096, 4097, 3*4096-5, 70001), every bit set, a transposed view."""
    from sdcguard_amd.serve_weights import fingerprint
    gen = torch.Generator().manual_seed(0)
    cases = []
    for n in (1, 7, 4096, 4097, 3 * 4096 - 5, 70001):
        if dt == torch.uint8:
            cases.append(torch.randint(0, 256, (n,), generator=gen, dtype=torch.uint8))
        else:
            cases.append((torch.randn(n, generator=gen) * 3).to(dt))
    es = torch.empty(0, dtype=dt).element_size()
    cases.append(torch.full((4096 + 3,), -1, dtype={1: torch.uint8, 2: torch.int16, 4: torch.int32,
                                                     8: torch.int64}[es]).view(dt))
    cases.append(torch.randn(96, 130, generator=gen).to(dt).t())
    for c in cases:
        got = _np(fingerprint(c.cuda()))
        want = F.fp2(F.fp2_words(_np(c.contiguous())))
        assert np.array_equal(got, want), (dt, tuple(c.shape))
        if c.numel() <= 200:
            assert tuple(got) == F.fp2_py(F.fp2_words(_np(c.contiguous())))
