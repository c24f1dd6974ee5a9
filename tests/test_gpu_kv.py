"""Paged-KV block fingerprints (sdc_kv_fingerprint through sdcguard_amd.kv) bit-exact against the oracle (fp3 of
each block's words from 0, the value recompute.fingerprint gives the block on its own) and against this library's
own whole-tensor fingerprint per block; the ledger check catches stale / reused blocks and K/V bit flips; the
28-layer x 4096-block Qwen3-0.6B-like cache with 64 sequences of 512-2048 tokens."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import fingerprint as F

pytestmark = pytest.mark.gpu


def _cache(nblocks, hkv=8, n=16, d=128, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(nblocks, hkv, n, 2 * d, device="cuda", generator=g).bfloat16()


def test_block_fingerprints_bit_exact():
    from sdcguard_amd.kv import block_fingerprints
    from sdcguard_amd.recompute import fingerprint
    cache = _cache(37, hkv=2, n=16, d=64)
    fp = block_fingerprints(cache).cpu().numpy()
    ref = F.kv_block_fp3(cache.view(torch.int16).cpu().numpy())
    assert np.array_equal(fp, ref)
    for b in (0, 5, 36):
        assert np.array_equal(fp[b], fingerprint(cache[b]).cpu().numpy())
    ids = torch.tensor([3, -1, 3, 36, 40, 0], device="cuda")
    fi = block_fingerprints(cache, ids).cpu().numpy()
    assert np.array_equal(fi[[0, 2, 3, 5]], ref[[3, 3, 36, 0]])
    assert not fi[[1, 4]].any()                              # no block: zeros


def test_odd_sized_and_strided_blocks():
    """Blocks whose word count is not a multiple of the per-thread slice, and blocks padded apart in memory."""
    from sdcguard_amd.kv import block_fingerprints
    g = torch.Generator(device="cuda").manual_seed(1)
    base = torch.randn(9, 3, 1000, device="cuda", generator=g).bfloat16()
    cache = base[:, :, :777]                                 # block b at stride 3000 words, 2331 words... per row gap
    blocks = torch.stack([cache[b].contiguous() for b in range(9)])
    fp = block_fingerprints(blocks).cpu().numpy()
    ref = F.kv_block_fp3(blocks.view(torch.int16).cpu().numpy())
    assert np.array_equal(fp, ref)
    padded = base[:, :2]                                     # each block 2000 contiguous words, 3000 apart
    fp2 = block_fingerprints(padded).cpu().numpy()
    ref2 = F.kv_block_fp3(padded.contiguous().view(torch.int16).cpu().numpy())
    assert np.array_equal(fp2, ref2)


def test_whole_chunk_blocks_extremes_and_padding():
    """Blocks of whole 128-byte chunks, 16-byte aligned (the int8 matrix-core kernel): 320 words (five chunks, so a
    workgroup's four waves take 2, 2, 1 and none), 64 and 32768 words (the table's limit), blocks of words at the
    int16 extremes, entry counts that are not multiples of 64, dead and repeated entries, blocks padded apart in
    memory (2048 words at a stride of 3072), and caches of 1-byte words at the int8 extremes."""
    from sdcguard_amd.kv import block_fingerprints
    g = torch.Generator(device="cuda").manual_seed(4)
    for words, nblk in ((320, 70), (64, 130), (32768, 67)):
        raw = torch.randint(-32768, 32768, (nblk, words), generator=g, device="cuda", dtype=torch.int32)
        raw = raw.to(torch.int16)
        raw[0] = -32768
        raw[1] = 32767
        raw[2] = 0
        ref = F.kv_block_fp3(raw.cpu().numpy())
        assert np.array_equal(block_fingerprints(raw).cpu().numpy(), ref), words
        ids = torch.tensor([nblk - 1, -1, 0, 1, nblk, 2, 0], device="cuda")
        fi = block_fingerprints(raw, ids).cpu().numpy()
        assert np.array_equal(fi[[0, 2, 3, 5, 6]], ref[[nblk - 1, 0, 1, 2, 0]]), words
        assert not fi[[1, 4]].any()
    base = torch.randn(9, 3, 1024, device="cuda", generator=g).bfloat16()
    padded = base[:, :2]
    ref = F.kv_block_fp3(padded.contiguous().view(torch.int16).cpu().numpy())
    assert np.array_equal(block_fingerprints(padded).cpu().numpy(), ref)
    # 1-byte words (int8): 128 (one chunk), 640 and 65536 (the table's limit) bytes a block, int8 extremes
    for words, nblk in ((128, 70), (640, 66), (65536, 65)):
        raw = torch.randint(-128, 128, (nblk, words), generator=g, device="cuda", dtype=torch.int32).to(torch.int8)
        raw[0] = -128
        raw[1] = 127
        ref = F.kv_block_fp3(raw.cpu().numpy())
        assert np.array_equal(block_fingerprints(raw).cpu().numpy(), ref), words
        ids = torch.tensor([nblk - 1, -1, 1, 0], device="cuda")
        fi = block_fingerprints(raw, ids).cpu().numpy()
        assert np.array_equal(fi[[0, 2, 3]], ref[[nblk - 1, 1, 0]]) and not fi[1].any(), words


def test_ledger_catches_stale_blocks_and_bit_flips():
    from sdcguard_amd.kv import KVLedger
    cache = _cache(64, hkv=4, n=16, d=64, seed=2)
    g = torch.Generator().manual_seed(3)
    bt = torch.randint(0, 64, (6, 10), generator=g).cuda()
    bt[2, 7:] = -1
    led = KVLedger(cache, 6, 10)
    led.record(bt)
    assert led.verify(bt).read()["mismatched"] == 0
    stale = bt.clone()
    stale[4, 3] = (bt[4, 3] + 1) % 64                        # the table points at another block
    r = led.verify(stale).read()
    assert r["entries"] == [(4, 3)] or (bt == stale[4, 3]).sum() > 0
    assert (4, 3) in r["entries"]
    blk = int(bt[1, 5])
    v = cache[blk, 2, 7, 100:101].view(torch.int16)
    v ^= 1 << 3                                              # one bit of one value of one block
    r = led.verify(bt).read()
    want = sorted(tuple(x) for x in (bt == blk).nonzero().cpu().tolist())
    assert sorted(r["entries"]) == want and r["mismatched"] == len(want)


def test_fp8_cache_block_fingerprints_bit_exact():
    """A cache of 1-byte elements (fp8 e4m3 keys and values) has int8 words (recompute.py:86-87): every block is
    bit-exact against the oracle and against this library's fingerprint of the block on its own, also with blocks
    whose byte count is not a multiple of a lane's 16 bytes and blocks 1 byte off alignment; a flipped bit changes
    its block's fingerprint only; the ledger over an fp8 cache flags a stale entry."""
    from sdcguard_amd.kv import KVLedger, block_fingerprints
    from sdcguard_amd.recompute import fingerprint
    g = torch.Generator(device="cuda").manual_seed(11)
    cache = (torch.randn(29, 4, 16, 128, device="cuda", generator=g) * 8).to(torch.float8_e4m3fn)
    fp = block_fingerprints(cache).cpu().numpy()
    ref = F.kv_block_fp3(cache.view(torch.int8).cpu().numpy())
    assert np.array_equal(fp, ref)
    for b in (0, 13, 28):
        assert np.array_equal(fp[b], fingerprint(cache[b]).cpu().numpy())
    base = (torch.randn(13, 2000, device="cuda", generator=g) * 8).to(torch.float8_e4m3fn)
    for view in (base[:, :777], base[:, 1:778], base[:, 3:2000]):
        got = block_fingerprints(view).cpu().numpy()
        want = F.kv_block_fp3(view.contiguous().view(torch.int8).cpu().numpy())
        assert np.array_equal(got, want), view.shape
    c2 = cache.clone()
    c2.view(torch.uint8)[3, 1, 5, 7] ^= 0x10
    fp2 = block_fingerprints(c2).cpu().numpy()
    assert (fp2 != fp).any(axis=1).nonzero()[0].tolist() == [3]
    bt = torch.tensor([[0, 5, 9, -1], [3, 3, 28, 7]], device="cuda")
    led = KVLedger(cache, 2, 4)
    led.record(bt)
    assert led.verify(bt).read()["mismatched"] == 0
    stale = bt.clone()
    stale[1, 2] = 27
    assert led.verify(stale).read()["entries"] == [(1, 2)]


def test_qwen3_like_cache_28_layers_4096_blocks():
    """28 layers x 4096 blocks of [8 KV heads, 16 tokens, 2 x 128] bf16 N(0,1) (7.5 GB); 64 sequences of U[512,
    2048] tokens whose block-table entries are drawn from the 4096 blocks with replacement (about 80 blocks a
    sequence: pages are shared); every fingerprint of a sample of 512 (layer, block) pairs is bit-exact against the
    oracle layer by layer (all 114,688); the ledger flags a stale entry and a flipped bit, exactly where they
    are."""
    from sdcguard_amd.kv import KVLedger, block_fingerprints
    layers, nblk = 28, 4096
    g = torch.Generator(device="cuda").manual_seed(11)
    cache = torch.empty(layers * nblk, 8, 16, 256, dtype=torch.bfloat16, device="cuda")
    for lay in range(layers):
        cache[lay * nblk:(lay + 1) * nblk] = torch.randn(nblk, 8, 16, 256, device="cuda", generator=g).bfloat16()
    fp = block_fingerprints(cache).cpu().numpy()
    rng = np.random.default_rng(12)
    if F.c_lib() is not None:
        # every block, one layer (256 MB) at a time, against the C restatement on the host's cores
        threads = min(16, os.cpu_count() or 1)
        for lay in range(layers):
            sub = cache[lay * nblk:(lay + 1) * nblk].view(torch.int16).cpu().numpy()
            ref = F.kv_block_fp3_c(sub, threads=threads)
            bad = np.nonzero((fp[lay * nblk:(lay + 1) * nblk] != ref).any(axis=1))[0]
            assert bad.size == 0, (lay, bad[:5])
        print(f"{layers * nblk} block fingerprints bit-exact against the C oracle")
    else:
        sample = rng.choice(layers * nblk, 512, replace=False)
        sub = cache[torch.from_numpy(sample).cuda()].view(torch.int16).cpu().numpy()
        assert np.array_equal(fp[sample], F.kv_block_fp3(sub))
    lens = rng.integers(512, 2049, 64)
    W = int(-(-lens.max() // 16))
    bt = torch.full((64, W), -1, dtype=torch.int64)
    for r, L in enumerate(lens):
        nb = int(-(-L // 16))
        bt[r, :nb] = torch.from_numpy(rng.integers(0, nblk, nb))
    bt = bt.cuda()
    layer = 17
    lc = cache[layer * nblk:(layer + 1) * nblk]
    led = KVLedger(lc, 64, W)
    led.record(bt)
    assert led.verify(bt).read()["mismatched"] == 0
    stale = bt.clone()
    stale[40, 10] = (int(bt[40, 10]) + 1234) % nblk
    r = led.verify(stale).read()
    assert (40, 10) in r["entries"]
    blk = int(bt[7, 3])
    v = lc[blk, 5, 9, 200:201].view(torch.int16)
    v ^= 1 << 14
    r = led.verify(bt).read()
    want = sorted(tuple(x) for x in (bt == blk).nonzero().cpu().tolist())
    assert sorted(r["entries"]) == want
