"""Write the golden fixtures of the floating-point checks from the reference itself.

Run once, in a container that has the reference checked out at /root/reference (never on a GPU box):

    SDCGUARD_SIGN_SEED=1 python tests/golden/make_golden.py [signs] [train] [serve] [quant]

It imports the reference's checksum and serve modules (pure Python + torch, CPU) and records, for seeded small
cases, the inputs and the reference's answers:
  * signs.npz      the epoch-0 sign table of widths 1..128 and the epoch-3 table (checksum._signs at seed 1);
  * train.npz      checksum.matmul_zscores + resolve: every checksum's score (the array the reference reduces
                   with torch.max, recorded on the way) and the resolved (max_z, batch, row, col_block, noise);
  * acc.npz        checksum.matmul_zscores_acc + resolve (the precise check of an fp32 output): the same records;
  * serve.npz      serve.check_static_impl: every checksum's score, the state row (keys and counts);
  * quant.npz      modes.judge on fp8 e4m3 and int8 GEMMs (inputs from modes._inputs, results of modes.gemm's CPU
                   path, with and without an injected fault): per-block z and wrong-block counts;
  * fused.npz      fused.fused_mm (output words, float64 block statistics), fused.zscores_from_stats on them (clean,
                   faults added to the accumulator, epoch 3, nfma) and fused.fused_mm_checked (scored in the kernel),
                   run in Triton's CPU interpreter (TRITON_INTERPRET=1 in the environment);
  * fp8.npz        serve_fp8.quant_check_torch (the FP8 quantization check): each recipe clean, scales taken over
                   padding rows or otherwise wrong, codes one, two and three steps off, a static scale changed,
                   non-finite inputs, an unarmed step, MoE rows per token; the state row after each case's calls;
  * weights.npz    serve_weights.model_digest and fingerprint of a small model with 1, 2, 4 and 8-byte parameters;
  * moe.npz        serve_moe.moe_check_torch (the sampled fused-MoE recompute): the state row and the kept row after
                   one call on the reference's verification scenarios and a larger routed-first case;
  * route.npz      serve_route.route_check_torch (the MoE router check) and serve_route.judge on every row: the
                   softmax, sigmoid, biased and grouped (DeepSeek) policies, fp32 / bf16 / fp16 logits, routing as
                   the policy gives it, a moved expert, a repeated expert, weights off, an id out of range, a
                   padding row, tied scores, an inactive step and a step without real rows: the state row, the kept
                   row and every row's (wrong set, wrong weight, weight differences);
  * attn.npz       serve_attn.attn_check_torch on make_case calls (shapes, request mixes, a sliding window, wrong
                   outputs, wrong KV writes and slots, block ids outside the cache, non-finite values, padding)
                   over several steps: every sample's per-dimension scores, the 18-column state row and the
                   capture row; sample_python's picks on a grid of batches; recheck on kept samples.
Only numbers are stored (inputs as raw 16-bit or 8-bit words).  The integer fingerprints need no fixture: closed
forms and brute force pin them (tests/test_oracle_fingerprint.py).
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

REF = os.environ.get("SDCGUARD_REFERENCE", "/root/reference/src")
OUT = os.path.dirname(os.path.abspath(__file__))


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


class _MaxRecorder:
    """Records the tensors passed to torch.max(t, 0) (the reference's reduction of every checksum's score)."""

    def __init__(self):
        self.seen = []
        self._orig = torch.max

    def __enter__(self):
        orig = self._orig

        def rec(*a, **kw):
            if len(a) == 2 and a[1] == 0 and isinstance(a[0], torch.Tensor) and a[0].dim() == 1:
                self.seen.append(a[0].detach().clone())
            return orig(*a, **kw)

        torch.max = rec
        return self

    def __exit__(self, *exc):
        torch.max = self._orig


def make_signs(cs):
    t0 = np.zeros((128, 128), np.float32)
    t3 = np.zeros((128, 128), np.float32)
    for w in range(1, 129):
        t0[w - 1, :w] = cs._signs(w, "cpu").numpy()
        t3[w - 1, :w] = cs._signs(w, "cpu", 3).numpy()
    np.savez_compressed(os.path.join(OUT, "signs.npz"), epoch0=t0, epoch3=t3, seed=np.int64(1))


def _train_cases():
    """(name, A, B, C, bias, alpha, beta, dtype) seeded cases: clean and corrupted, the shapes of _group._probe,
    bmm, remainder blocks, alpha/beta, 2-D bias, fp16, tiny and huge outputs, NaN/Inf."""
    g = torch.Generator().manual_seed(7)
    cases = []

    def r(*shape, dt=torch.bfloat16, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dt)

    shapes = [(96, 80, 300, True), (70, 48, 1500, False), (70, 48, 2600, True), (64, 96, 40, False),
              (48, 700, 300, True), (33, 130, 129, True), (5, 17, 1, False), (1, 64, 128, True)]
    spots = [(70, 140), (5, 1300), (66, 2599), (17, 39), (40, 250), (32, 128), (4, 0), (0, 77)]
    for dt in (torch.bfloat16, torch.float16):
        for (m, k, n, wb), spot in zip(shapes, spots):
            a, b = r(m, k, dt=dt), r(k, n, dt=dt, scale=1 / math.sqrt(k))
            bias = r(n, dt=dt) if wb else None
            c = torch.addmm(bias.float(), a.float(), b.float()).to(dt) if wb else (a.float() @ b.float()).to(dt)
            tag = f"{str(dt)[6:]}_{m}x{k}x{n}"
            cases.append((tag + "_clean", a, b, c, bias, 1.0, 1.0, dt))
            bad = c.clone()
            bad[spot] = bad[spot] + 50.0
            cases.append((tag + "_plus50", a, b, bad, bias, 1.0, 1.0, dt))
            bad = c.clone()
            bad[spot] = float("nan")
            cases.append((tag + "_nan", a, b, bad, bias, 1.0, 1.0, dt))
    # bmm (batch 2), shared-B bmm
    a, b = r(2, 40, 64), r(2, 64, 136, scale=0.125)
    c = torch.bmm(a.float(), b.float()).bfloat16()
    cases.append(("bf16_bmm_clean", a, b, c, None, 1.0, 1.0, torch.bfloat16))
    bad = c.clone()
    bad[1, 33, 130] += 50
    cases.append(("bf16_bmm_plus50", a, b, bad, None, 1.0, 1.0, torch.bfloat16))
    # alpha / beta with a 2-D bias (checksum tests: addmm with 2-D bias and scaling)
    a, b = r(64, 128), r(128, 256, scale=1 / math.sqrt(128))
    bias2 = r(64, 256)
    c = torch.addmm(bias2.float(), a.float(), b.float(), beta=0.5, alpha=2.0).bfloat16()
    cases.append(("bf16_addmm2d_clean", a, b, c, bias2, 2.0, 0.5, torch.bfloat16))
    bad = c.clone()
    bad[10, 32:64] = 0
    cases.append(("bf16_addmm2d_zeroed", a, b, bad, bias2, 2.0, 0.5, torch.bfloat16))
    # tiny outputs (no false alarm down to 1e-30) and a tiny value turned big
    W = r(256, 256, scale=0.02)
    for sc in (1e-18, 1e-24, 1e-30):
        dY = r(64, 256, scale=sc)
        dX = (dY.float() @ W.float()).bfloat16()
        cases.append((f"bf16_tiny{sc:g}_clean", dY, W, dX, None, 1.0, 1.0, torch.bfloat16))
    dY = r(64, 256, scale=1e-24)
    dX = (dY.float() @ W.float()).bfloat16()
    bad = dX.clone()
    bad[3, 5] = 1e-3
    cases.append(("bf16_tiny_to_big", dY, W, bad, None, 1.0, 1.0, torch.bfloat16))
    # Inf output, an Inf input (expected side not finite: unjudged), an exponent-bit flip
    a, b = r(32, 64), r(64, 256, scale=0.125)
    c = (a.float() @ b.float()).bfloat16()
    bad = c.clone()
    bad[7, 200] = float("inf")
    cases.append(("bf16_inf_out", a, b, bad, None, 1.0, 1.0, torch.bfloat16))
    ainf = a.clone()
    ainf[3, 3] = float("inf")
    cases.append(("bf16_inf_in", ainf, b, c, None, 1.0, 1.0, torch.bfloat16))
    bad = c.clone()
    v = bad.view(-1)[5000:5001].view(torch.int16)
    bad.view(-1)[5000] = (v ^ (1 << 14)).view(torch.bfloat16)[0]
    cases.append(("bf16_bit14", a, b, bad, None, 1.0, 1.0, torch.bfloat16))
    # fp16 overflow: huge outputs the inputs can produce (unjudged) vs. ones they cannot (a fault)
    a16, b16 = r(16, 64, dt=torch.float16, scale=200.0), r(64, 128, dt=torch.float16, scale=20.0)
    c16 = (a16.float() @ b16.float()).half()
    cases.append(("fp16_overflow", a16, b16, c16, None, 1.0, 1.0, torch.float16))
    # identical columns (B of ones): the plain sum's worst-case rule
    a = r(32, 64)
    b = torch.ones(64, 256, dtype=torch.bfloat16)
    c = (a.float() @ b.float()).bfloat16()
    cases.append(("bf16_ones_clean", a, b, c, None, 1.0, 1.0, torch.bfloat16))
    return cases


class _Store:
    """Arrays stored once: identical tensors share an entry, and a tensor that differs from an earlier one of its
    shape in a few elements (a corrupted copy of a clean output) is stored as (positions, new words) edits."""

    def __init__(self):
        self.out, self._seen, self._last = {}, {}, {}

    def put(self, t: torch.Tensor) -> str:
        b = _bits(t)
        key = (b.shape, b.tobytes())
        if key in self._seen:
            return self._seen[key]
        name = f"a{len(self._seen)}"
        base = self._last.get(b.shape)
        if base is not None:
            diff = np.nonzero(self.out_full[base].reshape(-1) != b.reshape(-1))[0]
            if diff.size <= 64:
                self.out[name + "_base"] = np.array(base)
                self.out[name + "_edit"] = np.stack([diff.astype(np.int64), b.reshape(-1)[diff].astype(np.int64)])
                self._seen[key] = name
                self.out_full[name] = b
                return name
        self.out[name] = b
        self.out_full[name] = b
        self._seen[key] = name
        self._last[b.shape] = name
        return name

    out_full: dict = {}


def make_train(cs):
    st_ = _Store()
    st_.out_full = {}
    out = st_.out
    names = []
    for i, (name, a, b, c, bias, alpha, beta, dt) in enumerate(_train_cases()):
        with _MaxRecorder() as mr:
            st = cs.matmul_zscores(a, b, c, bias, alpha=alpha, beta=beta)
        res = cs.resolve([st], 6.0)[0]
        names.append(name)
        p = f"c{i}_"
        out[p + "ids"] = np.array([st_.put(a), st_.put(b), st_.put(c), st_.put(bias) if bias is not None else ""])
        out[p + "shapes"] = np.array([list(a.shape) + [0] * (3 - a.dim()), list(b.shape) + [0] * (3 - b.dim()),
                                      list(c.shape) + [0] * (3 - c.dim()),
                                      (list(bias.shape) if bias is not None else []) + [0] * (3 - (bias.dim() if bias is not None else 0))],
                                     np.int64)
        out[p + "meta"] = np.array([alpha, beta, 1.0 if dt == torch.float16 else 0.0], np.float64)
        out[p + "zs"] = np.concatenate([z.numpy().astype(np.float32) for z in mr.seen])
        out[p + "result"] = np.array([res.max_z, -1 if res.batch is None else res.batch, res.row, res.col_block,
                                      res.noise], np.float64)
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(OUT, "train.npz"), **out)
    return len(names)


def _acc_cases():
    """Small products with an fp32 output: (name, A, B, C, bias, alpha, beta, nfma, epoch)."""
    g = torch.Generator().manual_seed(11)

    def r(*shape, dt=torch.bfloat16, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dt)

    cases = []
    for dt, tag in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        a, b = r(16, 256, dt=dt), r(256, 256, dt=dt, scale=0.05)
        c = a.float() @ b.float()
        cases.append((f"{tag}_clean", a, b, c, None, 1.0, 1.0, None, 0))
        cases.append((f"{tag}_clean_nfma16", a, b, c, None, 1.0, 1.0, 16, 0))
        bad = c.clone()
        bad[5, 77] = bad[5, 77] * (1 + 2.0 ** -10)
        cases.append((f"{tag}_rel_2e-10", a, b, bad, None, 1.0, 1.0, None, 0))
    a, b = r(24, 512), r(512, 300, scale=0.02)
    c = a.float() @ b.float()
    cases.append(("bf16_remainder_300", a, b, c, None, 1.0, 1.0, None, 0))
    bad = c.clone()
    bad[7, 290] += 0.01
    cases.append(("bf16_remainder_fault", a, b, bad, None, 1.0, 1.0, None, 0))
    a, b = r(3, 8, 64), r(3, 64, 200)
    cases.append(("bf16_bmm", a, b, a.float() @ b.float(), None, 1.0, 1.0, None, 0))
    b1 = r(64, 200)
    cases.append(("bf16_shared_b", a, b1, a.float() @ b1.float(), None, 1.0, 1.0, None, 0))
    a, b = r(12, 128), r(128, 384, scale=0.1)
    bias = r(384)
    c = 0.5 * (a.float() @ b.float()) + 2.0 * bias.float()
    cases.append(("bf16_bias_vec_alpha_beta", a, b, c, bias, 0.5, 2.0, None, 0))
    bm = r(12, 384)
    cases.append(("bf16_bias_mat", a, b, a.float() @ b.float() + bm.float(), bm, 1.0, 1.0, None, 0))
    cases.append(("bf16_epoch3", a, b, a.float() @ b.float(), None, 1.0, 1.0, None, 3))
    a, b = r(8, 2048), r(2048, 256, scale=0.02)
    c = a.float() @ b.float()
    cases.append(("bf16_k2048", a, b, c, None, 1.0, 1.0, 16, 0))
    for what, val in (("nan", float("nan")), ("inf", float("inf")), ("plus1", None)):
        bad = c.clone()
        bad[3, 130] = val if val is not None else bad[3, 130] + 1.0
        cases.append((f"bf16_{what}", a, b, bad, None, 1.0, 1.0, None, 0))
    from sdcguard import checksum as cs_
    s0 = cs_._signs(128, "cpu", 0)
    j = next(j for j in range(1, 128) if s0[j] == s0[0])
    bad = c.clone()
    bad[2, 0], bad[2, j] = 1e18, -1e18
    cases.append(("bf16_huge_cancel", a, b, bad, None, 1.0, 1.0, None, 0))
    an = a.clone()
    an[1] = float("nan")
    cases.append(("bf16_nan_row_unjudged", an, b, an.float() @ b.float(), None, 1.0, 1.0, None, 0))
    a0, b0 = r(4, 0), r(0, 256)
    cases.append(("bf16_k0", a0, b0, torch.zeros(4, 256), None, 1.0, 1.0, None, 0))
    for scale in (0.0, 1e-24):
        at = torch.full((3, 8), scale, dtype=torch.bfloat16)
        bt = torch.ones(8, 260, dtype=torch.bfloat16)
        cases.append((f"bf16_tiny_{scale:g}", at, bt, at.float() @ bt.float(), None, 1.0, 1.0, None, 0))
    return cases


def make_acc(cs):
    st_ = _Store()
    st_.out_full = {}
    out = st_.out
    names = []
    for i, (name, a, b, c, bias, alpha, beta, nfma, epoch) in enumerate(_acc_cases()):
        with _MaxRecorder() as mr:
            st = cs.matmul_zscores_acc(a, b, c, bias, alpha=alpha, beta=beta, nfma=nfma, epoch=epoch)
        res = cs.resolve([st], 6.0)[0]
        names.append(name)
        p = f"c{i}_"
        out[p + "ids"] = np.array([st_.put(a), st_.put(b), st_.put(c.view(torch.int32).view(torch.int16)),
                                   st_.put(bias) if bias is not None else ""])
        out[p + "shapes"] = np.array([list(a.shape) + [0] * (3 - a.dim()), list(b.shape) + [0] * (3 - b.dim()),
                                      list(c.shape) + [0] * (3 - c.dim()),
                                      (list(bias.shape) if bias is not None else []) + [0] * (3 - (bias.dim() if bias is not None else 0))],
                                     np.int64)
        out[p + "meta"] = np.array([alpha, beta, 1.0 if a.dtype == torch.float16 else 0.0, nfma or 0, epoch],
                                   np.float64)
        out[p + "zs"] = np.concatenate([z.numpy().astype(np.float32) for z in mr.seen])
        out[p + "result"] = np.array([res.max_z, -1 if res.batch is None else res.batch,
                                      -1 if res.row is None else res.row,
                                      -1 if res.col_block is None else res.col_block,
                                      float("nan") if res.noise is None else res.noise], np.float64)
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(OUT, "acc.npz"), **out)
    return len(names)


def _fused_operands(m, k, n, dtype, bias, layout, seed):
    """A (m, k), B (k, n), bias: a linear layer's forward (B = w.t(), w stored (n, k)), a plain B, or a weight
    gradient's A = gy.t() (gy stored (k, m))."""
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(m, k, generator=g).to(dtype)
    B = (torch.randn(k, n, generator=g) / max(k, 1) ** 0.5).to(dtype)
    if layout == "w.t()":
        B = B.t().contiguous().t()
    elif layout == "gy.t()":
        A = A.t().contiguous().t()
    b = (torch.randn(n, generator=g) * 0.5).to(dtype) if bias else None
    return A, B, b


FUSED_LAYOUTS = ("plain", "w.t()", "gy.t()")
FUSED_SHAPES = [(16, 96, 200, True, "w.t()"), (33, 64, 128, False, "plain"), (8, 40, 77, True, "w.t()"),
                (5, 256, 300, True, "gy.t()"), (70, 130, 129, False, "w.t()"), (1, 32, 256, True, "plain"),
                (300, 64, 520, True, "w.t()")]


def make_fused(fused, cs):
    """fused.fused_mm (output words and float64 block statistics), fused.zscores_from_stats on those statistics
    (clean, faults added to the accumulator, another epoch's pattern, nfma) and fused.fused_mm_checked (the fp32
    self-check scored in the kernel), all in Triton's CPU interpreter."""
    st_ = _Store()
    st_.out_full = {}
    out = st_.out
    names = []

    def rec(name, kind, A, B, b, layout, nfma=None, epoch=0, inject=None, stats=None, **res):
        i = len(names)
        names.append(name)
        p = f"c{i}_"
        out[p + "ids"] = np.array([st_.put(A.contiguous()), st_.put(B.contiguous()),
                                   st_.put(b) if b is not None else ""])
        iv = inject if inject is not None else (-1, -1, 0.0)
        out[p + "meta"] = np.array([1.0 if A.dtype == torch.float16 else 0.0, FUSED_LAYOUTS.index(layout),
                                    nfma or 0, epoch, iv[0], iv[1], iv[2], {"fm": 0, "zs": 1, "chk": 2}[kind]],
                                   np.float64)
        out[p + "shape"] = np.array([A.shape[0], A.shape[1], B.shape[1]], np.int64)
        if stats is not None:
            out[p + "stats"] = stats.numpy()
        for key, val in res.items():
            out[p + key] = val

    def resolved(st, seen):
        r = cs.resolve([st], 6.0)[0]
        zs = np.concatenate([z.numpy().astype(np.float32) for z in seen]) if seen else np.zeros(0, np.float32)
        row = np.array([r.max_z, -1 if r.row is None else r.row, -1 if r.col_block is None else r.col_block,
                        float("nan") if r.noise is None else r.noise], np.float64)
        return zs, row

    for dtype in (torch.bfloat16, torch.float16):
        tag = "bf16" if dtype == torch.bfloat16 else "fp16"
        for i, (m, k, n, bias, layout) in enumerate(FUSED_SHAPES):
            A, B, b = _fused_operands(m, k, n, dtype, bias, layout, i)
            base = f"{tag}_{m}x{k}x{n}_{layout}"
            C, stats = fused.fused_mm(A, B, b)
            rec(base + "_fm", "fm", A, B, b, layout, stats=stats, C=_bits(C))
            with _MaxRecorder() as mr:
                st = fused.zscores_from_stats(A, B, stats, b)
            zs, row = resolved(st, mr.seen)
            rec(base + "_zs", "zs", A, B, b, layout, stats=stats, zs=zs, result=row)
            row_i, col_i = m // 2, n - 1
            for delta in (1.0, 1e-2, float("inf"), float("nan")):
                inj = (row_i, col_i, delta) if math.isfinite(delta) else (0, 0, delta)
                _, st2 = fused.fused_mm(A, B, b, inject=inj)
                with _MaxRecorder() as mr:
                    st = fused.zscores_from_stats(A, B, st2, b)
                zs, row = resolved(st, mr.seen)
                rec(base + f"_zs_inj{delta:g}", "zs", A, B, b, layout, inject=inj, stats=st2, zs=zs, result=row)
            A2, B2, b2 = _fused_operands(m, k, n, dtype, bias, layout, 100 + i)
            with _MaxRecorder() as mr:
                C2, st = fused.fused_mm_checked(A2, B2, b2)
            zs, row = resolved(st, mr.seen)
            rec(base + "_chk", "chk", A2, B2, b2, layout, C=_bits(C2), zs=zs, result=row)
            typical = float(C2.float().abs().median()) or 1.0
            inj = (m - 1, n - 1, 0.01 * typical)
            with _MaxRecorder() as mr:
                _, st = fused.fused_mm_checked(A2, B2, b2, inject=inj)
            zs, row = resolved(st, mr.seen)
            rec(base + "_chk_inj", "chk", A2, B2, b2, layout, inject=inj, zs=zs, result=row)
    # another epoch's pattern and the tensor-core step count, on one bf16 case
    A, B, b = _fused_operands(32, 128, 256, torch.bfloat16, True, "w.t()", 99)
    _, st3 = fused.fused_mm(A, B, b, epoch=3)
    with _MaxRecorder() as mr:
        st = fused.zscores_from_stats(A, B, st3, b, epoch=3, nfma=16)
    zs, row = resolved(st, mr.seen)
    rec("bf16_epoch3_nfma16_zs", "zs", A, B, b, "w.t()", nfma=16, epoch=3, stats=st3, zs=zs, result=row)
    with _MaxRecorder() as mr:
        _, st = fused.fused_mm_checked(A, B, b, epoch=3, nfma=16)
    zs, row = resolved(st, mr.seen)
    rec("bf16_epoch3_nfma16_chk", "chk", A, B, b, "w.t()", nfma=16, epoch=3, zs=zs, result=row)
    # self-check: an Inf the inputs cannot produce, and an Inf input (unjudged)
    with _MaxRecorder() as mr:
        _, st = fused.fused_mm_checked(A, B, b, inject=(5, 7, float("inf")))
    zs, row = resolved(st, mr.seen)
    rec("bf16_chk_inf_acc", "chk", A, B, b, "w.t()", inject=(5, 7, float("inf")), zs=zs, result=row)
    A2 = A.clone()
    A2[3, 4] = float("inf")
    with _MaxRecorder() as mr:
        _, st = fused.fused_mm_checked(A2, B, b)
    zs, row = resolved(st, mr.seen)
    rec("bf16_chk_inf_input", "chk", A2, B, b, "w.t()", zs=zs, result=row)
    # fp16 weights whose block sums exceed fp16's range (the parts are scaled by a power of two)
    g = torch.Generator().manual_seed(0)
    A = torch.randn(16, 64, generator=g).half()
    B = (torch.rand(64, 256, generator=g) * 900 + 100).half()
    with _MaxRecorder() as mr:
        C, st = fused.fused_mm_checked(A, B)
    zs, row = resolved(st, mr.seen)
    rec("fp16_large_block_sums_chk", "chk", A, B, None, "plain", C=_bits(C), zs=zs, result=row)
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(OUT, "fused.npz"), **out)
    return len(names)


def _fp8_cases(sf):
    """serve_fp8.quant_check_torch calls: (name, x2, xq codes, xs, recipe, scale_ub, static_ref, real rows, steps,
    mult); each case's calls (one per step) add into one state row."""
    g = torch.Generator().manual_seed(5)
    out = []
    for dt, tag in ((torch.bfloat16, "bf16"), (torch.float16, "fp16"), (torch.float32, "fp32")):
        m, pad, k = 24, 8, 96
        x = (torch.randn(m + pad, k, generator=g) * 3).to(dt)
        x[m:] *= 20                                   # padding rows left by an earlier, larger request
        real = 19
        st = torch.tensor([17], dtype=torch.int64)
        rows = sf.sample_rows(st, torch.tensor([real]))
        # per tensor
        ok_s = (x[:real].float().abs().amax() / 448.0).reshape(1)
        xq = sf.quantize(x, ok_s, False)
        out.append((f"{tag}_tensor_clean", x, xq, ok_s, 1, None, None, real, [17], 1))
        out.append((f"{tag}_tensor_not_armed", x, xq, ok_s, 1, None, None, 0, [17], 1))
        pad_s = (x.float().abs().amax() / 448.0).reshape(1)
        out.append((f"{tag}_tensor_from_padding", x, sf.quantize(x, pad_s, False), pad_s, 1, None, None, real, [17],
                    1))
        out.append((f"{tag}_tensor_scale_wrong", x, sf.quantize(x, ok_s * 1.1, False), ok_s * 1.1, 1, None, None, real,
                    [17], 1))
        out.append((f"{tag}_tensor_rows_all", x, sf.quantize(x, pad_s, False), pad_s, 1, None, None, m + pad, [17], 1))
        for d, what in ((1, "one_step"), (2, "two_steps"), (-3, "three_steps_down")):
            bad = xq.clone()
            r = int(rows[1])
            bad[r, 5] = (bad[r, 5].to(torch.int32) + d).clamp(0, 126).to(torch.uint8) if bad[r, 5] < 0x80 else \
                (bad[r, 5].to(torch.int32) - d).clamp(0x80, 0xFE).to(torch.uint8)
            out.append((f"{tag}_tensor_values_{what}", x, bad, ok_s, 1, None, None, real, [17], 1))
        # per token
        tok = (x.float().abs().amax(-1, keepdim=True) / 448.0).clamp(min=sf.MIN_SCALE)
        xqt = sf.quantize(x, tok, True)
        out.append((f"{tag}_token_clean", x, xqt, tok, 2, None, None, real, [17, 18, 2 ** 32 + 5], 1))
        badt = tok.clone()
        badt[int(rows[0])] *= 1.5
        out.append((f"{tag}_token_scale_wrong", x, sf.quantize(x, badt, True), badt, 2, None, None, real, [17], 1))
        ub = torch.tensor([0.5 * float(x[:real].float().abs().max())])
        tub = (torch.minimum(x.float().abs().amax(-1, keepdim=True), ub) / 448.0).clamp(min=sf.MIN_SCALE)
        out.append((f"{tag}_token_ub", x, sf.quantize(x, tub, True), tub, 2, ub, None, real, [17, 21], 1))
        out.append((f"{tag}_token_ub_missing", x, sf.quantize(x, tub, True), tub, 2, None, None, real, [17], 1))
        out.append((f"{tag}_token_moe_mult2", x, xqt, tok, 2, None, None, 9, [33, 34], 2))
        # static
        s0 = torch.tensor([0.02])
        xqs = sf.quantize(x, s0, False)
        out.append((f"{tag}_static_clean", x, xqs, s0, 0, None, s0.clone(), real, [17], 1))
        out.append((f"{tag}_static_changed", x, xqs, s0, 0, None, torch.tensor([0.021]), real, [17, 40], 1))
        out.append((f"{tag}_static_no_ref", x, xqs, s0, 0, None, None, real, [17], 1))
        # non-finite input in a sampled row
        xn = x.clone()
        xn[int(rows[0]), 7] = float("nan")
        out.append((f"{tag}_tensor_nan_input", xn, xq, ok_s, 1, None, None, real, [17], 1))
        xi = x.clone()
        xi[int(rows[0]), 9] = float("inf")
        out.append((f"{tag}_token_inf_input", xi, sf.quantize(xi, tok, True), tok, 2, None, None, real, [17], 1))
    return out


def make_fp8(sf):
    """serve_fp8.quant_check_torch: each case's state row after its calls."""
    st_ = _Store()
    st_.out_full = {}
    out = st_.out
    names = []
    for i, (name, x, xq, xs, recipe, ub, sref, real, steps, mult) in enumerate(_fp8_cases(sf)):
        state = torch.zeros(1, sf.COLS, dtype=torch.int64)
        rows_buf = torch.tensor([real], dtype=torch.int64)
        for stp in steps:
            sf.quant_check_torch(x, xq, xs, recipe, ub, sref, rows_buf, torch.tensor([stp], dtype=torch.int64),
                                 state, 0, mult)
        names.append(name)
        p = f"c{i}_"
        out[p + "ids"] = np.array([st_.put(x), st_.put(xq.view(torch.int8).to(torch.int16))])
        dtc = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 4}[x.dtype]
        out[p + "meta"] = np.array([dtc, recipe, real, mult, x.shape[0], x.shape[1], xq.shape[0]], np.int64)
        out[p + "steps"] = np.array(steps, np.int64)
        out[p + "xs"] = xs.float().reshape(-1).numpy()
        out[p + "ub"] = np.array([] if ub is None else ub.float().reshape(-1).tolist(), np.float32)
        out[p + "sref"] = np.array([] if sref is None else sref.float().reshape(-1).tolist(), np.float32)
        out[p + "state"] = state[0].numpy()
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(OUT, "fp8.npz"), **out)
    return len(names)


def digest_model():
    """A small model with parameters of every element size the fingerprint takes (2, 4 and 8 bytes, and 1 byte
    for an int8 parameter), as (name, tensor) in a fixed order."""
    g = torch.Generator().manual_seed(9)
    return [("a.weight", (torch.randn(96, 64, generator=g)).bfloat16()),
            ("a.bias", torch.randn(96, generator=g).bfloat16()),
            ("b.weight", torch.randn(33, 96, generator=g).half()),
            ("c.scale", torch.randn(7, 5, generator=g)),
            ("d.table", torch.randn(4, 3, generator=g).double()),
            ("e.q", torch.randint(-128, 128, (40, 8), generator=g, dtype=torch.int8))]


def make_weights(sw):
    """serve_weights.model_digest and fingerprint of digest_model()'s parameters (the PyTorch version, CPU)."""
    params = digest_model()
    model = torch.nn.Module()
    for name, t in params:
        mod_name, attr = name.split(".")
        if not hasattr(model, mod_name):
            model.add_module(mod_name, torch.nn.Module())
        getattr(model, mod_name).register_parameter(attr, torch.nn.Parameter(t, requires_grad=False))
    out = {"digest": np.array(sw.model_digest(model)), "names": np.array([n for n, _ in params])}
    for name, t in params:
        out["fp_" + name] = sw.fingerprint(t).numpy()
        out["bits_" + name] = t.contiguous().view(-1).view(torch.uint8).numpy()
    np.savez_compressed(os.path.join(OUT, "weights.npz"), **out)
    return len(params)


def make_moe(sm):
    """serve_moe.moe_check_torch: the state row and the kept row after one call, on the reference's own verification
    scenarios (serve_moe.py:524-598: clean, a wrong output, an expert map with a missing expert, an inactive step,
    a padding row, garbage past the step's real rows, a real row unrouted or partly routed), for SiLU and GELU in bf16
    and SiLU in fp16, plus a larger routed-first case with a wrong routing weight and a NaN output."""
    st_ = _Store()
    st_.out_full = {}
    out = st_.out
    names = []

    def rec(name, x, y, g, ids, w13, w2, emap, act, rf, raw, nl, idx):
        m, H = x.shape
        k = ids.shape[1]
        state = torch.zeros(1, sm.COLS, dtype=torch.int64)
        cm = torch.zeros(1, sm.CAP_COLS, dtype=torch.int32)
        cx, cy = torch.zeros(1, H), torch.zeros(1, H)
        ci, cg = torch.zeros(1, max(k, 8), dtype=torch.int64), torch.zeros(1, max(k, 8))
        sb = torch.full((1,), raw, dtype=torch.int64)
        sm.moe_check_torch(x, y, g, ids, w13, w2, emap, act, rf, state, 0, sb, nl, idx, cm, cx, cy, ci, cg, sm.MOE_Z)
        i = len(names)
        names.append(name)
        p = f"c{i}_"
        out[p + "ids"] = np.array([st_.put(x), st_.put(y), st_.put(w13), st_.put(w2)])
        out[p + "topk"] = ids.numpy().astype(np.int32)
        out[p + "g"] = g.float().numpy()
        out[p + "emap"] = np.array([] if emap is None else emap.tolist(), np.int32)
        out[p + "meta"] = np.array([1 if x.dtype == torch.float16 else 0, act, int(rf), raw, nl, idx,
                                    int(emap is not None)], np.int64)
        out[p + "state"] = state[0].numpy()
        out[p + "cap"] = cm[0].numpy().astype(np.int64)
        out[p + "cap_x"], out[p + "cap_y"] = cx[0].numpy(), cy[0].numpy()
        out[p + "cap_ids"], out[p + "cap_g"] = ci[0, :k].numpy(), cg[0, :k].numpy()

    for dtype, act, tag in ((torch.bfloat16, 0, "bf16_silu"), (torch.bfloat16, 1, "bf16_gelu"),
                            (torch.float16, 0, "fp16_silu")):
        gen = torch.Generator().manual_seed(0)
        E, H, I, K, M = 6, 192, 96, 3, 5
        w13 = (torch.randn(E, 2 * I, H, generator=gen) * 0.05).to(dtype)
        w2 = (torch.randn(E, H, I, generator=gen) * 0.05).to(dtype)
        x = torch.randn(M, H, generator=gen).to(dtype)
        g, ids = torch.topk(torch.softmax(torch.randn(M, E, generator=gen), -1), K, -1)
        ids = ids.to(torch.int32)
        emap = torch.tensor([0, 1, -1, 2, 3, 4], dtype=torch.int32)
        w13m, w2m = w13[:5].contiguous(), w2[:5].contiguous()
        ids_pad = ids.clone()
        ids_pad[M - 1] = -1
        ids_part = ids.clone()
        ids_part[1, 0] = -1
        for case in ("clean", "wrong", "map", "inactive", "padding", "real_rows", "unrouted_real", "partial_real"):
            step = 3 if case != "inactive" else 4
            given = {"real_rows": 3, "unrouted_real": M, "partial_real": M}.get(case)
            raw = sm.pack_step(step, given)
            use_map = case == "map"
            cids = ids_pad if case in ("padding", "unrouted_real") else ids_part if case == "partial_real" else ids
            y = sm._reference_layer(x, cids, g, w13m if use_map else w13, w2m if use_map else w2,
                                    emap if use_map else None, act, dtype)
            if case == "wrong":
                rows = sm.sample_rows(torch.tensor(step), M, "cpu", 4)
                y[int(rows[0]), 17] = y[int(rows[0]), 17] * 4 + 1
            elif case in ("padding", "unrouted_real"):
                y[M - 1] = 1000.0
            elif case == "real_rows":
                y[3:] = 1000.0
            rec(f"{tag}_{case}", x, y, g, cids, w13m if use_map else w13, w2m if use_map else w2,
                emap if use_map else None, act, False, raw, 4, 3)
    # larger, routing weight applied on the input
    gen = torch.Generator().manual_seed(1)
    E, H, I, K, M = 8, 256, 128, 4, 40
    w13 = (torch.randn(E, 2 * I, H, generator=gen) * 0.04).bfloat16()
    w2 = (torch.randn(E, H, I, generator=gen) * 0.04).bfloat16()
    x = torch.randn(M, H, generator=gen).bfloat16()
    g, ids = torch.topk(torch.softmax(torch.randn(M, E, generator=gen), -1), K, -1)
    ids = ids.to(torch.int32)
    y = sm.recompute(x, ids, g, w13, w2, None, 0, True, torch.bfloat16)[0].to(torch.bfloat16)
    raw = sm.pack_step(10, 33)
    rows = sm.sample_rows(torch.tensor(10), torch.tensor(33), "cpu", 2)
    rec("bf16_routed_first_clean", x, y, g, ids, w13, w2, None, 0, True, raw, 2, 0)
    g2 = g.clone()
    g2[int(rows[1]), 2] *= 1.25
    y2 = sm.recompute(x, ids, g2, w13, w2, None, 0, True, torch.bfloat16)[0].to(torch.bfloat16)
    rec("bf16_routed_first_wrong_weight", x, y2, g, ids, w13, w2, None, 0, True, raw, 2, 0)
    y3 = y.clone()
    y3[int(rows[0]), 100] = float("nan")
    rec("bf16_routed_first_nan_output", x, y3, g, ids, w13, w2, None, 0, True, raw, 2, 0)
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(OUT, "moe.npz"), **out)
    return len(names)


ROUTE_POLICIES = {
    # name: (E, k, scoring (0 softmax, 1 sigmoid), renormalize, bias, groups, topk_group, scale)
    "softmax_top4": (64, 4, 0, True, False, 0, 0, 1.0),
    "sigmoid_top6": (64, 6, 1, False, False, 0, 0, 1.0),
    "biased_top4": (64, 4, 1, True, True, 0, 0, 1.5),
    "deepseek_grouped": (256, 8, 1, True, True, 8, 4, 2.5),
    "grouped_softmax": (64, 6, 0, False, False, 4, 2, 1.0),
    "grouped_small_groups": (96, 4, 1, True, True, 12, 3, 1.0),
}


def make_route(sr):
    """serve_route.route_check_torch on seeded router calls (8 rows; state, kept row) and serve_route.judge on every
    row of the same call (fp32 logits as the check computes them)."""
    st_ = _Store()
    out = st_.out
    names = []
    for pname, (E, k, scoring, renorm, has_bias, groups, tg, scale) in ROUTE_POLICIES.items():
        for dtype in (torch.float32, torch.bfloat16, torch.float16):
            gen = torch.Generator().manual_seed(len(names) + 7)
            M = 8
            bias = (torch.randn(E, generator=gen) * 0.03) if has_bias else None
            lg = (torch.randn(M, E, generator=gen) * 2.0).to(dtype)
            w, ids = sr._reference_route(lg.float(), k, scoring, renorm, bias, groups, tg, scale)
            cases = ["clean", "moved_expert", "repeated_expert", "weights_off", "weights_within", "id_out_of_range",
                     "padding", "inactive", "no_rows"]
            if dtype == torch.float32 and not groups:
                cases.append("ties")
            for case in cases:
                lg_c, w_c, ids_c = lg.clone(), w.clone(), ids.clone()
                step, real = 5, M
                if case == "moved_expert":
                    ids_c[:, -1] = lg.float().argmin(-1).to(ids_c.dtype)
                elif case == "repeated_expert":
                    ids_c[:, 1] = ids_c[:, 0]
                elif case == "weights_off":
                    w_c[:, 0] *= 1.02
                elif case == "weights_within":
                    w_c = w_c * (1 + 3e-6)
                elif case == "id_out_of_range":
                    ids_c[:, 0] = E + 3
                elif case == "padding":
                    ids_c[:] = -1
                elif case == "inactive":
                    step = 6
                elif case == "no_rows":
                    real = 0
                elif case == "ties":
                    lg_c = torch.zeros(M, E)
                    lg_c[:, 0] = 3.0
                    w_c, ids_c = sr._reference_route(lg_c, k, scoring, renorm, bias, groups, tg, scale)
                    ids_c[:, 1] = (ids_c[:, 1] + 7) % E                 # another of the tied experts
                    ids_c[:, 1] = torch.where(ids_c[:, 1] == 0, torch.ones_like(ids_c[:, 1]), ids_c[:, 1])
                    s_ = torch.softmax(lg_c, -1) if scoring == 0 else torch.sigmoid(lg_c)
                    ww = s_.gather(1, ids_c.long())
                    w_c = ((ww / ww.sum(-1, keepdim=True)) if renorm else ww) * scale
                state = torch.zeros(1, sr.COLS, dtype=torch.int64)
                caps = sr.new_caps("cpu", 1, E)
                rb = torch.full((1,), real, dtype=torch.int64)
                sb = torch.full((1,), step, dtype=torch.int64)
                sr.route_check_torch(lg_c, w_c, ids_c, k, scoring, renorm, bias, groups, tg, scale, rb, sb, state, 0,
                                     2, 1, *caps)
                u = sr.unit_roundoff(lg_c.dtype)
                sb_all, wb_all, diff_all = sr.judge(lg_c.float(), ids_c.long(), w_c.float(), k, scoring, renorm,
                                                    bias, groups, tg, scale, u)
                i = len(names)
                names.append(f"{pname}_{str(dtype).replace('torch.', '')}_{case}")
                p = f"c{i}_"
                if dtype == torch.float32:
                    out[p + "logits"] = lg_c.numpy()
                else:
                    out[p + "logits_bits"] = _bits(lg_c)
                out[p + "ids"] = ids_c.numpy().astype(np.int32)
                out[p + "w"] = w_c.float().numpy()
                out[p + "bias"] = bias.numpy() if bias is not None else np.zeros(0, np.float32)
                out[p + "meta"] = np.array([E, k, scoring, int(renorm), groups, tg, {torch.float32: 0,
                                            torch.bfloat16: 1, torch.float16: 2}[dtype], step, real, 2, 1], np.int64)
                out[p + "scale"] = np.float32(scale)
                out[p + "state"] = state[0].numpy()
                out[p + "cap_meta"] = caps[0][0].numpy()
                out[p + "cap_lg"] = caps[1][0].numpy()
                out[p + "cap_ids"] = caps[2][0, :k].numpy()
                out[p + "cap_w"] = caps[3][0, :k].numpy()
                out[p + "set_bad"] = sb_all.numpy()
                out[p + "w_bad"] = wb_all.numpy()
                out[p + "diff"] = diff_all.float().numpy()
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(OUT, "route.npz"), **out)
    return len(names)


def _serve_cases():
    g = torch.Generator().manual_seed(11)
    shapes = [(64, 256, 300, True), (1, 256, 1000, False), (200, 96, 40, True), (33, 130, 129, True),
              (300, 64, 700, False), (64, 192, 1100, True), (16, 256, 512, False), (40, 128, 128, True)]
    cases = []
    for dt in (torch.bfloat16, torch.float16):
        for m, k, n, wb in shapes:
            W = (torch.randn(n, k, generator=g) / k ** 0.5).to(dt)
            b = torch.randn(n, generator=g).to(dt) if wb else None
            x = torch.randn(m, k, generator=g).to(dt)
            y = torch.nn.functional.linear(x.float(), W.float(), None if b is None else b.float()).to(dt)
            tag = f"{str(dt)[6:]}_{m}x{k}x{n}"
            cases.append((tag + "_clean", x, W, b, y, dt))
            rr, cc = (m * 2) // 3, (n * 3) // 5
            bad = y.clone()
            bad[rr, cc] = bad[rr, cc] + 50.0
            cases.append((tag + "_plus50", x, W, b, bad, dt))
            bad = y.clone()
            bad[rr, cc] = float("nan")
            cases.append((tag + "_nan", x, W, b, bad, dt))
            bad = y.clone()
            bad[rr, cc] = float("inf")
            cases.append((tag + "_inf", x, W, b, bad, dt))
    # an input that is not finite: every checksum of its row is unjudged
    W = (torch.randn(256, 64, generator=g) / 8).bfloat16()
    x = torch.randn(8, 64, generator=g).bfloat16()
    y = (x.float() @ W.float().t()).bfloat16()
    x2 = x.clone()
    x2[2, 5] = float("inf")
    cases.append(("bf16_inf_input", x2, W, None, y, torch.bfloat16))
    # tiny outputs
    W = (torch.randn(384, 128, generator=g) * 0.02).bfloat16()
    x = (torch.randn(32, 128, generator=g) * 1e-24).bfloat16()
    y = (x.float() @ W.float().t()).bfloat16()
    cases.append(("bf16_tiny", x, W, None, y, torch.bfloat16))
    return cases


def make_serve(sv):
    st_ = _Store()
    st_.out_full = {}
    out = st_.out
    names = []
    for i, (name, x, W, b, y, dt) in enumerate(_serve_cases()):
        cs = sv.LayerChecksums(W, b, 128)
        state = torch.zeros(1, sv.STATE_COLS, dtype=torch.int64)
        with _MaxRecorder() as mr:
            sv.check_static_impl(x, y, *cs.tensors(True), state, 0, 6.0, 1e-20)
        names.append(name)
        p = f"c{i}_"
        out[p + "ids"] = np.array([st_.put(x), st_.put(W), st_.put(y), st_.put(b) if b is not None else ""])
        out[p + "shape"] = np.array([x.shape[0], x.shape[1], W.shape[0]], np.int64)
        out[p + "dtype"] = np.int64(1 if dt == torch.float16 else 0)
        out[p + "zs"] = mr.seen[0].numpy().astype(np.float32)[:-1]       # (the appended 0 dropped)
        out[p + "state"] = state[0].numpy().copy()
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(OUT, "serve.npz"), **out)
    return len(names)


def make_quant(md):
    """modes.judge on small fp8 and int8 GEMMs (the fp8 unit and products per step of an unknown GPU).  Per input
    set: a, b, the clean result c, and for each fault (none, +small, +large, NaN, huge; int8: none, +1) the changed
    element (row, col, value), the per-block z and the wrong-block count."""
    out = {}
    i = 0
    gen = torch.Generator().manual_seed(11)
    for mode in ("fp8", "int8"):
        for shape in ((24, 256, 256), (9, 384, 384)):
            for dist, scale in (md.VARIANTS[:4] if shape[0] == 24 else md.VARIANTS[:2]):
                a, b, a64, b64 = md._inputs(mode, shape, dist, scale, gen)
                c0 = md.gemm(mode, a, b)
                if mode == "fp8":
                    out[f"q{i}_a"] = a.view(torch.uint8).numpy().copy()
                    out[f"q{i}_b"] = b.view(torch.uint8).numpy().copy()
                else:
                    out[f"q{i}_a"] = a.numpy().copy()
                    out[f"q{i}_b"] = b.numpy().copy()
                out[f"q{i}_c"] = c0.numpy().copy()
                out[f"q{i}_name"] = np.array(f"{mode} {shape} {dist} {scale}")
                faults = (None, "add") if mode == "int8" else (None, "add", "big", "nan", "huge")
                for f, fault in enumerate(faults):
                    c = c0.clone()
                    r = int(torch.randint(0, shape[0], (1,), generator=gen))
                    j = int(torch.randint(0, shape[2], (1,), generator=gen))
                    if fault is None:
                        pass
                    elif mode == "int8":
                        c[r, j] += 1
                    elif fault == "add":
                        blk = c[r, (j // 128) * 128:(j // 128 + 1) * 128].double()
                        c[r, j] += float(blk.norm() / math.sqrt(128)) * 0.02 + 1e-3
                    elif fault == "big":
                        blk = c[r, (j // 128) * 128:(j // 128 + 1) * 128].double()
                        c[r, j] += float(blk.norm() / math.sqrt(128)) * 0.5 + 1e-2
                    elif fault == "nan":
                        c[r, j] = float("nan")
                    else:
                        c[r, j] = 3e30
                    res = md.judge(mode, a64, b64, c, nfma=16, unit=md.UNIT["fp8"]) if mode == "fp8" else \
                        md.judge(mode, a64, b64, c)
                    out[f"q{i}_f{f}_at"] = np.array([r, j], np.int64)
                    out[f"q{i}_f{f}_v"] = np.array(c[r, j].item(), c0.numpy().dtype)
                    out[f"q{i}_f{f}_z"] = res["z"].float().numpy()
                    out[f"q{i}_f{f}_wrong"] = np.int64(res["wrong_blocks"])
                out[f"q{i}_nf"] = np.int64(len(faults))
                i += 1
    np.savez_compressed(os.path.join(OUT, "quant.npz"), **out)
    return i


class _NanToNumRecorder:
    """Records the per-dimension score vectors the reference's attention check passes through torch.nan_to_num (one
    call per sample, valid or not)."""

    def __init__(self):
        self.seen = []
        self._orig = torch.nan_to_num

    def __enter__(self):
        orig = self._orig

        def rec(t, *a, **kw):
            r = orig(t, *a, **kw)
            self.seen.append(r.detach().clone())
            return r

        torch.nan_to_num = rec
        return self

    def __exit__(self, *exc):
        torch.nan_to_num = self._orig


def _attn_cases(sa):
    """(name, case, left, runs) cases built with the reference's make_case (serve_attn.py:621-664): shapes, request
    mixes, a sliding window, and the faults its tests use (a wrong output, a wrong KV write, a block id outside the
    cache, a write to another slot, non-finite outputs and keys).  runs: (step, nl, idx, active) calls."""
    out = []
    steps = [(s, 1, 0, True) for s in range(6)]
    turns = [(s, 3, 1, True) for s in range(5)] + [(4, 1, 0, False)]
    lens_mix = ((70, 1), (21, 6), (3, 3), (0, 0))
    for dt in (torch.bfloat16, torch.float16):
        tag = "bf16" if dt == torch.bfloat16 else "fp16"
        for D, Hq, Hkv in ((64, 4, 2), (128, 2, 1), (128, 16, 8)):
            base = sa.make_case("cpu", dt, D=D, Hq=Hq, Hkv=Hkv, lens=lens_mix, seed=D + Hq)
            out.append((f"{tag}_D{D}_H{Hq}x{Hkv}_clean", base, -1, steps + turns))
            wrong = dict(base, o=base["o"].clone())
            wrong["o"][:, 1 % Hq, 5] = wrong["o"][:, 1 % Hq, 5].float() * 3 + 1
            out.append((f"{tag}_D{D}_H{Hq}x{Hkv}_wrong", wrong, -1, steps))
            if D == 64:
                badw = dict(base, key=base["key"].clone())
                badw["key"][:, 0, 3] = badw["key"][:, 0, 3].float() + 1
                out.append((f"{tag}_D{D}_badwrite", badw, -1, steps))
                badv = dict(base, val=base["val"].clone())
                badv["val"][:, Hkv - 1, D - 2] = badv["val"][:, Hkv - 1, D - 2].float() * -1 + 0.5
                out.append((f"{tag}_D{D}_badvalue", badv, -1, steps))
                badblk = dict(base, bt=base["bt"].clone())
                badblk["bt"][0, 1] = 10 ** 6
                out.append((f"{tag}_D{D}_badblock", badblk, -1, steps))
                negblk = dict(base, bt=base["bt"].clone())
                negblk["bt"][1, 0] = -1
                out.append((f"{tag}_D{D}_negblock", negblk, -1, steps))
                badslot = dict(base, slots=base["slots"].clone())
                badslot["slots"][:] = torch.where(badslot["slots"] >= 0, (badslot["slots"] + 1) % (12 * 16),
                                                  badslot["slots"])
                out.append((f"{tag}_D{D}_badslot", badslot, -1, steps))
                nano = dict(base, o=base["o"].clone())
                nano["o"][:, :, 7] = float("nan")
                out.append((f"{tag}_D{D}_nan_out", nano, -1, steps))
                infk = dict(base, kv=base["kv"].clone())
                infk["kv"][:, :, :, 9] = float("inf")
                out.append((f"{tag}_D{D}_inf_key", infk, -1, steps))
                out.append((f"{tag}_D{D}_window20", base, 20, steps))
        long_ = sa.make_case("cpu", dt, D=128, Hq=8, Hkv=2, NB=40, lens=((300, 1), (129, 1), (17, 4), (0, 0)),
                             seed=5, padded_rows=2)
        out.append((f"{tag}_long_clean", long_, -1, steps))
        lw = dict(long_, o=long_["o"].clone())
        lw["o"][:, 3, 100] = lw["o"][:, 3, 100].float() + 0.25
        out.append((f"{tag}_long_wrong", lw, -1, steps))
        out.append((f"{tag}_long_window7", long_, 7, steps[:3]))
        pad = sa.make_case("cpu", dt, D=64, Hq=2, Hkv=1, NB=4, lens=((0, 0), (0, 0)), seed=6, padded_rows=3)
        out.append((f"{tag}_all_padding", pad, -1, steps[:2]))
    return out


def make_attn(sa):
    """serve_attn.attn_check_torch on make_case calls over several steps, each from fresh buffers: every sample's
    per-dimension scores, the 18-column state row, the capture row and its q / o rows; sample_python's picks on a
    grid; recheck on kept samples."""
    st_ = _Store()
    st_.out_full = {}
    out = st_.out
    names = []
    for ci, (name, c, left, runs) in enumerate(_attn_cases(sa)):
        p = f"c{ci}_"
        D = c["q"].shape[-1]
        out[p + "ids"] = np.array([st_.put(c[k]) for k in ("q", "o", "kv", "key", "val")])
        out[p + "shape_q"] = np.array(c["q"].shape, np.int64)
        out[p + "shape_kv"] = np.array(c["kv"].shape, np.int64)
        out[p + "dtype"] = np.int64(1 if c["q"].dtype == torch.float16 else 0)
        out[p + "qsl"] = c["qsl"].numpy().astype(np.int64)
        out[p + "seq_lens"] = c["seq_lens"].numpy().astype(np.int64)
        out[p + "bt"] = c["bt"].numpy().astype(np.int64)
        out[p + "slots"] = c["slots"].numpy().astype(np.int64)
        out[p + "scale"] = np.float64(c["scale"])
        out[p + "left"] = np.int64(left)
        out[p + "runs"] = np.array([[s, nl, idx, int(a)] for s, nl, idx, a in runs], np.int64)
        for ri, (step, nl, idx, active) in enumerate(runs):
            b = sa.buffers("cpu", 1, D, 128, c["q"].dtype)
            with _NanToNumRecorder() as rec:
                sa.run_case(sa.attn_check_torch, c, b, step=step, nl=nl, idx=idx, left=left, active=active)
            q = f"{p}r{ri}_"
            out[q + "state"] = b["state"][0].numpy().copy()
            out[q + "capm"] = b["capm"][0].numpy().astype(np.int64)
            out[q + "capq"] = b["capq"][0, :D].numpy().copy()
            out[q + "capo"] = b["capo"][0, :D].numpy().copy()
            out[q + "z"] = torch.stack([z.float() for z in rec.seen]).numpy()
        names.append(name)
    out["names"] = np.array(names)
    # sample_python on a grid of batches (every kind of request mix, padding rows and requests)
    grid = []
    batches = [([0, 1, 7, 10, 10], [70, 21, 3, 0], 12, 4), ([0, 1, 2, 3, 4], [512, 900, 1500, 2047], 4, 16),
               ([0, 5, 5, 6], [5, 0, 40], 9, 8), ([0, 0], [0], 3, 2), ([0, 3], [3], 3, 2),
               ([0, 1, 2], [10, 20], 5, 32)]
    for bi, (qsl, sls, rows, heads) in enumerate(batches):
        for step in range(0, 41, 3):
            for nl, idx in ((1, 0), (3, 2), (28, 5)):
                for j in range(8):
                    s = sa.sample_python(step, idx, nl, j, qsl, sls, rows, heads)
                    v = [-1] * 5 if s is None else [s["row"], s["request"], s["position"], s["seq_len"], s["head"]]
                    grid.append([bi, step, nl, idx, j, *v])
    out["pick_grid"] = np.array(grid, np.int64)
    for bi, (qsl, sls, rows, heads) in enumerate(batches):
        out[f"pick_b{bi}"] = np.array([*qsl, -7, *sls, -7, rows, heads], np.int64)
    # recheck (float64) on rows of the long case, right and wrong
    c = sa.make_case("cpu", torch.bfloat16, D=128, Hq=8, Hkv=2, NB=40, lens=((300, 1), (129, 1)), seed=9)
    g = torch.Generator().manual_seed(3)
    for ri in range(4):
        r = ri % 2
        pos = int(c["seq_lens"][r]) - 1
        i = int(c["qsl"][r + 1]) - 1
        hq = ri * 2 + 1
        N = c["kv"].shape[2]
        rows = torch.stack([c["kv"][int(c["bt"][r, t // N]), hq // 4, t % N] for t in range(pos + 1)])
        o_row = c["o"][i, hq].float().clone()
        if ri >= 2:
            o_row[int(torch.randint(0, 128, (1,), generator=g))] += 0.5 * (ri - 1)
        res = sa.recheck(c["q"][i, hq], o_row, rows[:, :128], rows[:, 128:], c["scale"], torch.bfloat16)
        out[f"rc{ri}_q"] = _bits(c["q"][i, hq])
        out[f"rc{ri}_o"] = o_row.numpy().copy()
        out[f"rc{ri}_kv"] = _bits(rows)
        out[f"rc{ri}_scale"] = np.float64(c["scale"])
        out[f"rc{ri}_res"] = np.array([res["worst_score"], res["outputs_over_line"], res.get("dim", -1),
                                       res.get("output", 0.0), res.get("expected", 0.0),
                                       1.0 if res["verdict"] == "output_wrong" else 0.0])
    np.savez_compressed(os.path.join(OUT, "attn.npz"), **out)
    return len(names)


def main():
    if os.environ.get("SDCGUARD_SIGN_SEED") != "1":
        sys.exit("run with SDCGUARD_SIGN_SEED=1")
    sys.path.insert(0, REF)
    from sdcguard import checksum as cs
    from sdcguard import modes as md
    from sdcguard import serve as sv
    cs.USE_FAST = False
    torch.set_num_threads(4)
    which = sys.argv[1:] or ["signs", "train", "acc", "serve", "quant", "attn", "fused", "fp8", "weights", "moe",
                             "route"]
    if "route" in which:
        from sdcguard import serve_route as sr
        print("route.npz:", make_route(sr), "cases")
    if "moe" in which:
        from sdcguard import serve_moe as sm
        print("moe.npz:", make_moe(sm), "cases")
    if "weights" in which:
        from sdcguard import serve_weights as sw
        print("weights.npz:", make_weights(sw), "parameters")
    if "fp8" in which:
        from sdcguard import serve_fp8 as sf
        print("fp8.npz:", make_fp8(sf), "cases")
    if "fused" in which:
        if os.environ.get("TRITON_INTERPRET") != "1":
            sys.exit("fused.npz runs the reference's Triton kernels in the CPU interpreter: set TRITON_INTERPRET=1")
        from sdcguard import fused
        print("fused.npz:", make_fused(fused, cs), "cases")
    if "attn" in which:
        from sdcguard import serve_attn as sa
        print("attn.npz:", make_attn(sa), "cases")
    if "signs" in which:
        make_signs(cs)
    if "train" in which:
        print("train.npz:", make_train(cs), "cases")
    if "acc" in which:
        print("acc.npz:", make_acc(cs), "cases")
    if "serve" in which:
        print("serve.npz:", make_serve(sv), "cases")
    if "quant" in which:
        print("quant.npz:", make_quant(md), "cases")


if __name__ == "__main__":
    main()
