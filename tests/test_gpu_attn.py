"""The sampled attention recompute on the GPU (sdc_attn_check, through the C ABI) against the reference's own
outputs (tests/golden/attn.npz: serve_attn.attn_check_torch) and the oracle (oracle/attn.py): counts exactly,
every judged sample's per-dimension scores within 1e-3 of the reference's (relative, or absolute below 1), the
located alarm exactly.  Then the KV-cache geometry of a Qwen3-0.6B-like model (28 layers x 4096 blocks of
[8 KV heads, 16 tokens, 2 x 128] bf16, 64 decode sequences of 512-2048 tokens) with stale blocks and K/V bit flips:
verdicts must agree with the oracle on every fault."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn as OA
from tests._golden import load, names, words

pytestmark = pytest.mark.gpu

F = load("attn.npz")
NAMES = names(F)
COUNT_COLS = [OA.C_CALLS, OA.C_SAMPLES, OA.C_SKIP, OA.C_UNJ, OA.C_BADBLK, OA.C_KEYS, OA.C_WN, OA.C_WBAD,
              OA.C_WSLOT, OA.C_WLAST, OA.C_WWHERE]
DEV = torch.device("cuda", 0)


def zbits(key) -> float:
    return float(np.array([int(key) >> 32], np.uint32).view(np.float32)[0])


def _t16(w: np.ndarray, dt) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(w).astype(np.uint16).view(np.int16)).view(dt)


def fixture_case(ci):
    p = f"c{ci}_"
    dt = torch.float16 if int(F[p + "dtype"]) else torch.bfloat16
    q, o, kv, key, val = (_t16(words(F, str(n)), dt).to(DEV) for n in F[p + "ids"])
    return {"q": q, "o": o, "kv": kv, "key": key, "val": val,
            "qsl": torch.from_numpy(F[p + "qsl"]).to(torch.int32).to(DEV),
            "seq_lens": torch.from_numpy(F[p + "seq_lens"]).to(torch.int32).to(DEV),
            "bt": torch.from_numpy(F[p + "bt"]).to(torch.int32).to(DEV),
            "slots": torch.from_numpy(F[p + "slots"]).to(DEV),
            "scale": float(F[p + "scale"]), "left": int(F[p + "left"]), "runs": F[p + "runs"]}


def run_gpu(c, b, *, step, nl=1, idx=0, active=True, samples=None, left=None):
    from sdcguard_amd import serve_attn as SA
    ns = samples or b["samples"]
    zs = torch.full((ns, c["q"].shape[-1]), float("nan"), dtype=torch.float32, device=DEV)
    SA.run_case(c, b, step=step, nl=nl, idx=idx, active=active, left=c["left"] if left is None else left,
                scores_out=zs)
    torch.cuda.synchronize()
    return b["state"][0].cpu().numpy(), b["capm"][0].cpu().numpy().astype(np.int64), zs.cpu().numpy()


def oracle_of(c, step, nl=1, idx=0, active=True, samples=OA.SAMPLES, left=None):
    dt = "fp16" if c["q"].dtype == torch.float16 else "bf16"
    f = lambda t: t.float().cpu().numpy()                                    # noqa: E731
    return OA.check(f(c["q"]), f(c["o"]), f(c["kv"]), f(c["key"]), f(c["val"]), c["qsl"].cpu().numpy(),
                    c["seq_lens"].cpu().numpy(), c["bt"].cpu().numpy(), c["slots"].cpu().numpy(), step=step,
                    nl=nl, idx=idx, active=active, scale=c["scale"], left=c["left"] if left is None else left,
                    dtype=dt, samples=samples, kernel_keys=True)


def compare(state, capm, zs, want_state, want_z, samples_info, what):
    """GPU state / scores against the reference's (or the oracle's) for one call; returns the largest |dz|."""
    assert state[COUNT_COLS].tolist() == np.asarray(want_state)[COUNT_COLS].tolist(), (what, state, want_state)
    worst = 0.0
    for s in samples_info:
        if not s.judged:
            continue
        zr = np.asarray(want_z[s.j], np.float64)
        zg = zs[s.j].astype(np.float64)
        fin = np.isfinite(zr)
        assert np.array_equal(np.isfinite(zg), fin), (what, s.j)
        d = np.abs(zg[fin] - zr[fin])
        rel = d / np.maximum(1.0, zr[fin])
        assert (rel <= 1e-3).all(), (what, s.j, float(rel.max()))
        worst = max(worst, float(rel.max(initial=0.0)))
    zw, zg_ = zbits(want_state[OA.C_ZT]), zbits(state[OA.C_ZT])
    assert zw == zg_ or abs(zw - zg_) <= 1e-3 * max(1.0, zw), (what, zw, zg_)
    if zw > OA.ATTN_Z:
        for col in (OA.C_ZT, OA.C_ZH, OA.C_ZD, OA.C_ZS, OA.C_ZP):
            assert int(state[col]) & OA.M32 == int(want_state[col]) & OA.M32, (what, col)
    over = [s for s in samples_info if s.judged and s.zmax > OA.ATTN_Z]
    assert bool(capm[OA.CM_CLAIM]) == bool(over), what
    if len(over) == 1:                           # one candidate: the same sample kept
        s = over[0]
        assert capm[[OA.CM_ROW, OA.CM_HEAD, OA.CM_REQ, OA.CM_POS, OA.CM_SL, OA.CM_LO, OA.CM_DIM]].tolist() == \
            [s.row, s.head, s.request, s.position, s.seq_len, s.lo, s.dim], what
    return worst


@pytest.mark.parametrize("ci", range(len(NAMES)), ids=NAMES)
def test_matches_the_reference_check(ci):
    from sdcguard_amd import serve_attn as SA
    c = fixture_case(ci)
    worst = 0.0
    for ri, (step, nl, idx, active) in enumerate(c["runs"]):
        b = SA.buffers(DEV, 1, c["q"].shape[-1], 128, c["q"].dtype)
        st, cm, zs = run_gpu(c, b, step=int(step), nl=int(nl), idx=int(idx), active=bool(active))
        info = oracle_of(c, int(step), int(nl), int(idx), bool(active)).samples      # which samples are judged
        worst = max(worst, compare(st, cm, zs, F[f"c{ci}_r{ri}_state"], F[f"c{ci}_r{ri}_z"], info,
                                   f"{NAMES[ci]} run {ri}"))
        if cm[OA.CM_CLAIM] and sum(s.judged and s.zmax > OA.ATTN_Z for s in info) == 1:
            D = c["q"].shape[-1]
            assert np.array_equal(b["capq"][0, :D].cpu().numpy(), F[f"c{ci}_r{ri}_capq"], equal_nan=True)
            assert np.array_equal(b["capo"][0, :D].cpu().numpy(), F[f"c{ci}_r{ri}_capo"], equal_nan=True)
    print(f"{NAMES[ci]}: max relative |dz| vs the reference {worst:.2e}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lens,samples,D,heads", [
    (((4000, 1), (2500, 3), (700, 1), (0, 0)), 4, 128, (8, 2)),      # long contexts: many splits per sample
    (((1500, 1), (33, 1), (900, 2)), 16, 64, (4, 4)),
    (((257, 1), (256, 1), (255, 1), (17, 17)), 8, 256, (2, 1)),       # head size 256, tile boundaries
    (((100, 5), (60, 1)), 6, 80, (4, 2)),                            # a head size that is not a power of two
])
def test_matches_the_oracle_on_long_contexts(dtype, lens, samples, D, heads):
    from sdcguard_amd import serve_attn as SA
    Hq, Hkv = heads
    nblk = sum(-(-sl // 16) for sl, _ in lens)
    c = SA.make_case(DEV, dtype, D=D, Hq=Hq, Hkv=Hkv, NB=nblk + 3, lens=lens, seed=D + samples, padded_rows=2)
    c["left"] = -1
    wrong = dict(c, o=c["o"].clone())
    wrong["o"][:, Hq - 1, D // 3] = wrong["o"][:, Hq - 1, D // 3].float() * 1.5 + 0.3
    worst = 0.0
    for cc, tag in ((c, "clean"), (wrong, "wrong")):
        for step in range(4):
            b = SA.buffers(DEV, 1, D, 4096, dtype, samples=samples)
            st, cm, zs = run_gpu(cc, b, step=step, samples=samples)
            o = oracle_of(cc, step, samples=samples)
            zw = [s.z if s.z is not None else np.zeros(D) for s in o.samples]
            worst = max(worst, compare(st, cm, zs, o.state, zw, o.samples, f"{tag} step {step}"))
            if tag == "clean":
                assert zbits(st[OA.C_ZT]) <= 1.0              # a correct output scores at most 1
    print(f"max relative |dz| vs the oracle {worst:.2e}")


def test_one_workspace_serves_calls_of_any_context_length_and_sample_count():
    """A buffer reused by calls whose split counts and sample counts differ (the per-sample counters sit at fixed
    places and every call leaves them at zero): each call's state equals a call on fresh buffers."""
    from sdcguard_amd import serve_attn as SA
    cases = [SA.make_case(DEV, torch.bfloat16, D=128, Hq=4, Hkv=2, NB=nb, lens=lens, seed=i)
             for i, (nb, lens) in enumerate([(300, ((4000, 1), (700, 1))), (8, ((60, 1), (30, 2))),
                                              (120, ((1800, 1), (33, 1)))])]
    for c in cases:
        c["left"] = -1
        c["o"][:, 1, 9] += 0.75
    shared = SA.buffers(DEV, 1, 128, 64, torch.bfloat16, samples=32)
    for rep in range(2):
        for ci, c in enumerate(cases):
            for samples in (4, 32, 8):
                shared["state"].zero_()
                shared["capm"].zero_()
                shared["samples"] = samples
                SA.run_case(c, shared, step=rep * 5 + ci, keep_kv=False)
                fresh = SA.buffers(DEV, 1, 128, 64, torch.bfloat16, samples=samples)
                SA.run_case(c, fresh, step=rep * 5 + ci, keep_kv=False)
                torch.cuda.synchronize()
                assert torch.equal(shared["state"], fresh["state"]), (rep, ci, samples)
                assert int(shared["state"][0, OA.C_CALLS]) == 1
                assert int(shared["state"][0, OA.C_SAMPLES] + shared["state"][0, OA.C_SKIP] +
                           shared["state"][0, OA.C_UNJ] + shared["state"][0, OA.C_BADBLK]) == samples
    ws = shared["ws"]
    assert int(ws[:4096].view(torch.int32).abs().sum()) == 0          # the counters are back at zero


def test_keeps_the_attended_keys_and_the_recheck_confirms():
    from sdcguard_amd import serve_attn as SA
    c = SA.make_case(DEV, torch.bfloat16, D=128, Hq=4, Hkv=2, NB=30, lens=((300, 1), (90, 1)), seed=3)
    c["left"] = -1
    c["o"][:, :, 11] += 0.5
    b = SA.buffers(DEV, 1, 128, 512, torch.bfloat16)
    st, cm, _ = run_gpu(c, b, step=0)
    assert cm[OA.CM_CLAIM] == 1 and cm[OA.CM_KEPT] == 1
    kvm = b["capkvm"].cpu().tolist()
    assert kvm[0] == 1 and kvm[1] == 0 and kvm[2] == cm[OA.CM_POS] - cm[OA.CM_LO] + 1 and kvm[3] == 0
    r, pos, hk = int(cm[OA.CM_REQ]), int(cm[OA.CM_POS]), int(cm[OA.CM_HK])
    t = torch.arange(pos + 1, device=DEV)
    rows = c["kv"][c["bt"][r, t // 16].long(), hk, t % 16]
    kept = b["capkv"][:pos + 1]
    assert torch.equal(kept[:, 0, :128], rows[:, :128]) and torch.equal(kept[:, 1, :128], rows[:, 128:])
    res = SA.recheck(b["capq"][0, :128], b["capo"][0, :128], kept[:, 0, :128], kept[:, 1, :128], c["scale"],
                     torch.bfloat16)
    assert res["verdict"] == "output_wrong" and res["dim"] == 11
    ref = OA.recheck(b["capq"][0, :128].cpu().numpy(), b["capo"][0, :128].cpu().numpy(),
                     kept[:, 0, :128].float().cpu().numpy(), kept[:, 1, :128].float().cpu().numpy(), c["scale"],
                     "bf16")
    assert abs(res["worst_score"] - ref["worst_score"]) <= 1e-9 * ref["worst_score"]


def test_an_inactive_or_other_layers_step_counts_nothing():
    from sdcguard_amd import serve_attn as SA
    c = SA.make_case(DEV, torch.bfloat16)
    c["left"] = -1
    for kw in ({"active": False}, {"nl": 3, "idx": 1, "step": 3}):
        b = SA.buffers(DEV, 1, 64, 16, torch.bfloat16)
        kw = {"step": 0, **kw}
        SA.run_case(c, b, **kw)
        torch.cuda.synchronize()
        assert int(b["state"].abs().sum()) == 0 and int(b["capm"].abs().sum()) == 0


def test_graph_replays_match_eager_calls():
    """The check in a captured HIP graph (fixed buffers, no memset nodes): each replay, with the step set outside
    the graph and eager work in between, gives what an eager call gives."""
    from sdcguard_amd import serve_attn as SA
    c = SA.make_case(DEV, torch.bfloat16, D=128, Hq=8, Hkv=2, NB=60, lens=((600, 1), (300, 4), (5, 1)), seed=8)
    c["left"] = -1
    c["o"][:, 2, 40] += 1.0
    b = SA.buffers(DEV, 1, 128, 64, torch.bfloat16)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        SA.run_case(c, b, step=0)                         # warm (loads the library, first launch)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        SA.attn_check(c["q"], c["o"], c["kv"], c["key"], c["val"], c["qsl"], c["seq_lens"], c["bt"], c["slots"],
                      b["state"], 0, b["ctrl"], 1, 0, c["scale"], -1, SA.ATTN_Z, b["capm"], b["capq"], b["capo"],
                      b["capkv"], b["capkvm"], b["ws"], True, False)
    for step in range(6):
        for k in ("state", "capm"):
            b[k].zero_()
        b["ctrl"][0] = step
        b["ctrl"][1] = 1
        g.replay()
        torch.cuda.synchronize()
        got = b["state"][0].cpu().clone()
        e = SA.buffers(DEV, 1, 128, 64, torch.bfloat16)
        SA.run_case(c, e, step=step, keep_kv=False)
        torch.cuda.synchronize()
        assert torch.equal(got, e["state"][0].cpu()), step
        _ = torch.randn(1000, device=DEV).sum().item()    # eager work between replays


# ------------------------------------------------------------------- the full KV-cache geometry with faults
L_LAYERS, NBLK, HKV, NTOK, D, HQ, NSEQ = 28, 4096, 8, 16, 128, 16, 64


def _c5_cache():
    """28 layers x 4096 blocks x [8, 16, 256] bf16 ~ N(0,1) (7.5 GB), 64 sequences of 512-2048 tokens.  Block ids
    are drawn per sequence without repeats inside it; sequences may share blocks (they need ~5,100 blocks of the
    4,096), as prefix-shared blocks do."""
    g = torch.Generator(device=DEV).manual_seed(55)
    kv = torch.empty(L_LAYERS, NBLK, HKV, NTOK, 2 * D, dtype=torch.bfloat16, device=DEV)
    for layer in range(L_LAYERS):
        kv[layer].normal_(generator=g)
    gc = torch.Generator().manual_seed(56)
    lens = torch.randint(512, 2049, (NSEQ,), generator=gc)
    W = 2048 // NTOK
    bt = torch.zeros(NSEQ, W, dtype=torch.int32)
    for r in range(NSEQ):
        nb = -(-int(lens[r]) // NTOK)
        bt[r, :nb] = torch.randperm(NBLK, generator=gc)[:nb].to(torch.int32)
    q = (torch.randn(L_LAYERS, NSEQ, HQ, D, generator=gc) * 0.5).bfloat16().to(DEV)
    return kv, lens.to(torch.int32), bt, q


def _decode_outputs(kv_l, bt, lens, q_l):
    """A correct backend's outputs for one layer's decode step: fp32 attention of each sequence's query over its
    keys (positions 0..seq_len-1 through the block table), rounded to bf16."""
    W = bt.shape[1]
    blocks = kv_l[bt.to(DEV).long()]                                        # [seqs, W, Hkv, 16, 2D]
    rows = blocks.permute(0, 1, 3, 2, 4).reshape(NSEQ, W * NTOK, HKV, 2 * D).float()
    K, V = rows[..., :D], rows[..., D:]
    qf = q_l.float().view(NSEQ, HKV, HQ // HKV, D)
    s = torch.einsum("bkhd,bhgd->bhgk", K, qf) * D ** -0.5
    live = torch.arange(W * NTOK, device=DEV)[None, :] < lens.to(DEV)[:, None]
    s = s.masked_fill(~live[:, None, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bhgk,bkhd->bhgd", p, V).reshape(NSEQ, HQ, D).bfloat16()


def _compact_for_oracle(kv_l, bt, slots, rows_used):
    """The blocks the sampled requests can read (their block-table rows and their slots), remapped, so the oracle
    sees the same keys without copying the whole cache."""
    ids = sorted({int(v) for r in rows_used for v in bt[r].tolist() if 0 <= v < NBLK} |
                 {int(slots[r]) // NTOK for r in rows_used if 0 <= int(slots[r]) < NBLK * NTOK})
    remap = {b: i for i, b in enumerate(ids)}
    bt_c = bt.clone()
    for r in range(bt.shape[0]):
        bt_c[r] = torch.tensor([remap.get(int(v), 0) for v in bt[r].tolist()], dtype=torch.int32)
    sl_c = slots.clone()
    for r in range(slots.shape[0]):
        s = int(slots[r])
        if s // NTOK in remap:
            sl_c[r] = remap[s // NTOK] * NTOK + s % NTOK
    w = kv_l[torch.tensor(ids, device=DEV)].view(torch.int16).cpu().numpy().view(np.uint16)
    return (w.astype(np.uint32) << 16).view(np.float32), bt_c.numpy(), sl_c.numpy()


def test_kv_cache_geometry_with_stale_blocks_and_bit_flips():
    from sdcguard_amd import serve_attn as SA
    kv, lens, bt, q = _c5_cache()
    qsl = torch.arange(NSEQ + 1, dtype=torch.int32)
    pos = lens - 1
    blk_of = bt[torch.arange(NSEQ), (pos // NTOK).long()]
    slots = (blk_of.long() * NTOK + pos % NTOK).to(torch.int64)
    samples = 16              # 1/64 of the 64 decode rows x 16 heads per layer call
    scale = D ** -0.5
    bufs = SA.buffers(DEV, L_LAYERS, D, 4096, torch.bfloat16, samples=samples)
    g = torch.Generator().manual_seed(57)
    outcomes = {"clean": 0, "stale": [0, 0, 0], "flip": [0, 0, 0]}
    worst_clean = 0.0
    for layer in range(L_LAYERS):
        kv_l = kv[layer]
        o = _decode_outputs(kv_l, bt, lens, q[layer])
        key = kv_l[blk_of.long().to(DEV), :, (pos % NTOK).long().to(DEV), :D].contiguous()
        val = kv_l[blk_of.long().to(DEV), :, (pos % NTOK).long().to(DEV), D:].contiguous()
        step = layer * 7
        picks = [OA.sample(step, 0, 1, j, qsl.tolist(), lens.tolist(), NSEQ, HQ) for j in range(samples)]
        rows_used = sorted({p_["request"] for p_ in picks if p_})
        fault = ("clean", "stale", "flip")[layer % 3]
        o_sup, kv_chk = o, kv_l
        undo = None
        if fault == "stale":
            # the backend read a stale block for one sampled row: its output came from another block's keys
            r0 = picks[int(torch.randint(0, samples, (1,), generator=g))]["request"]
            nb = -(-int(lens[r0]) // NTOK)
            bt_bad = bt.clone()
            bt_bad[r0, int(torch.randint(0, nb, (1,), generator=g))] = int(torch.randint(0, NBLK, (1,), generator=g))
            o_sup = _decode_outputs(kv_l, bt_bad, lens, q[layer])
        elif fault == "flip":
            # a high exponent bit of K or V flips, after the backend ran, in a block that a sample attends with
            # the KV head it reads
            pk = picks[int(torch.randint(0, samples, (1,), generator=g))]
            r0, hk0 = pk["request"], pk["head"] // (HQ // HKV)
            nb = -(-int(lens[r0]) // NTOK)
            bi = int(bt[r0, int(torch.randint(0, nb, (1,), generator=g))])
            tk, dd = (int(torch.randint(0, n, (1,), generator=g)) for n in (NTOK, 2 * D))
            bit = int(torch.randint(12, 15, (1,), generator=g))
            w = kv_l[bi, hk0, tk, dd].view(torch.int16)
            undo = (bi, hk0, tk, dd, kv_l[bi, hk0, tk, dd].clone())
            kv_l[bi, hk0, tk, dd] = (w ^ (1 << bit)).view(torch.bfloat16)
        c = {"q": q[layer], "o": o_sup, "kv": kv_chk, "key": key, "val": val, "qsl": qsl.to(DEV),
             "seq_lens": lens.to(DEV), "bt": bt.to(DEV), "slots": slots.to(DEV), "scale": scale}
        zs = torch.full((samples, D), float("nan"), device=DEV)
        bufs["ctrl"][0], bufs["ctrl"][1] = step, 1
        SA.attn_check(c["q"], c["o"], c["kv"], c["key"], c["val"], c["qsl"], c["seq_lens"], c["bt"], c["slots"],
                      bufs["state"], layer, bufs["ctrl"], 1, 0, scale, -1, SA.ATTN_Z, bufs["capm"], bufs["capq"],
                      bufs["capo"], None, None, bufs["ws"], True, False, samples=samples, scores_out=zs)
        torch.cuda.synchronize()
        st = bufs["state"][layer].cpu().numpy()
        # the oracle on the same data (only the blocks the sampled requests can read)
        kv_c, bt_c, sl_c = _compact_for_oracle(kv_chk, bt, slots, rows_used)
        f = lambda t: t.float().cpu().numpy()                        # noqa: E731
        ora = OA.check(f(c["q"]), f(o_sup), kv_c, f(key), f(val), qsl.numpy(), lens.numpy(), bt_c, sl_c, step=step,
                       scale=scale, samples=samples, kernel_keys=True)
        zw = [s.z if s.z is not None else np.zeros(D) for s in ora.samples]
        compare(st, bufs["capm"][layer].cpu().numpy().astype(np.int64), zs.cpu().numpy(), ora.state, zw,
                ora.samples, f"layer {layer} {fault}")
        flagged = zbits(st[OA.C_ZT]) > SA.ATTN_Z
        assert flagged == (zbits(ora.state[OA.C_ZT]) > OA.ATTN_Z), (layer, fault)
        assert int(st[OA.C_WN]) == sum(1 for s in ora.samples if s.write_checked)
        if fault == "clean":
            assert not flagged
            worst_clean = max(worst_clean, zbits(st[OA.C_ZT]))
            outcomes["clean"] += 1
        else:
            outcomes[fault][0] += 1
            outcomes[fault][1] += int(flagged)
            outcomes[fault][2] += int(st[OA.C_UNJ] > 0)
        if undo is not None:
            bi, hk0, tk, dd, v = undo
            kv_l[bi, hk0, tk, dd] = v
    print(f"clean layers {outcomes['clean']} (worst score {worst_clean:.3f}); stale blocks flagged "
          f"{outcomes['stale'][1]}/{outcomes['stale'][0]}, K/V bit flips flagged {outcomes['flip'][1]}/"
          f"{outcomes['flip'][0]} (a non-finite sample, not judged: {outcomes['flip'][2]}); every verdict and count "
          "agrees with the oracle")
    del kv
    torch.cuda.empty_cache()
