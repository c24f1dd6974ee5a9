"""Sampled attention recompute from a paged KV cache, and the KV-write check (oracle: test infrastructure only).

Restates serve_attn.py of the reference:
  constants            :73-92   (ATTN_Z, SAMPLES, the sample-picking primes, the 18-column state row, CAPM)
  dtype_consts         serve_norm.py:69-77 (unit roundoff and output spacing of bf16 / fp16)
  p_spacing            :106-109
  bound_consts         :115-118
  sample               :130-157 (`sample_python`)
  check                :165-280 (`attn_check_torch`: one call, every sample, the state row, the capture, the
                                 KV-write check)
  recheck              :764-798 (float64 recompute of a kept sample)

Arithmetic follows the reference: scores, softmax and the bound in float32 (the reference's torch ops on fp32
tensors), the recheck in float64.  `check` also returns every sample's per-dimension scores (the vector the
reference reduces with `z.max(0)`), which the GPU tests compare element by element.

Where the reference's PyTorch check and its Triton kernels differ, `check` follows the PyTorch check unless told
otherwise: a judged sample whose every score is exactly 0 leaves the state's score keys alone in the kernels
(`if pz > 0.0`, serve_attn.py:481) but writes keys with a zero score in the PyTorch check (:241); `kernel_keys=True`
takes the kernels' rule.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

f32 = np.float32
M32 = 0xFFFFFFFF
S31 = 0x7FFFFFFF                                  # serve_norm.py:93
ATTN_Z = 4.0                                      # serve_attn.py:73
SAMPLES = 4                                       # :75
PICK_A, PICK_B, PICK_C = 1000003, 7919, 104729    # :85
TWO22, TWO21, TWO23 = 2.0 ** -22, 2.0 ** -21, 2.0 ** -23
COLS = 18                                         # :87-89
(C_ZT, C_ZH, C_ZD, C_ZO, C_ZR, C_ZS, C_ZP, C_CALLS, C_SAMPLES, C_SKIP, C_UNJ, C_BADBLK, C_KEYS, C_WN, C_WBAD,
 C_WSLOT, C_WLAST, C_WWHERE) = range(COLS)
CAPM = 12                                         # :90-91
(CM_CLAIM, CM_ROW, CM_HEAD, CM_REQ, CM_POS, CM_SL, CM_LO, CM_STEP, CM_Z, CM_KEPT, CM_DIM, CM_HK) = range(CAPM)
W_CONTENT, W_SLOT = 1, 2                          # :93


def dtype_consts(dtype: str):
    """(unit roundoff, output spacing) of the output dtype (serve_norm.py:69-77)."""
    if dtype == "fp16":
        return 2.0 ** -11, 2.0 ** -24
    return 2.0 ** -8, 1e-37


def p_spacing(dtype: str) -> float:
    """serve_attn.py:106-109."""
    return 2.0 ** -25 if dtype == "fp16" else 2.0 ** -126


def bound_consts(dtype: str, head_size: int):
    """(u, output spacing, P spacing, q.k accumulation coefficient): serve_attn.py:115-118."""
    u, sp = dtype_consts(dtype)
    return u, sp, p_spacing(dtype), (head_size + 8) * TWO23


def _first_at_least(arr, n, x) -> int:
    """The smallest k in [0, n] with arr[k] >= x, n when none is (torch.searchsorted / _lower_bound)."""
    for k in range(n + 1):
        if int(arr[k]) >= x:
            return k
    return n


def sample(step: int, idx: int, nl: int, j: int, qsl, seq_lens, rows: int, heads: int) -> Optional[dict]:
    """Sample j of the layer with index idx of nl at a step: serve_attn.py:130-157 (`sample_python`)."""
    nreq = len(seq_lens)
    ntok = min(int(qsl[nreq]), rows)
    h = (step // nl) * PICK_A + j * PICK_B + idx * PICK_C
    if ntok <= 0:
        return None
    if j % 2 == 0:
        pk = h % (ntok * heads)
        i = pk // heads
    else:
        rreal = _first_at_least(qsl, nreq, ntok)
        if rreal <= 0:
            return None
        pk = h % (rreal * heads)
        i = int(qsl[pk // heads + 1]) - 1
    r = _first_at_least(qsl, nreq, i + 1) - 1
    q0, q1, sl = int(qsl[r]), int(qsl[r + 1]), int(seq_lens[r])
    qlen = q1 - q0
    pos = sl - qlen + (i - q0)
    if not (0 <= i < rows and qlen > 0 and sl > 0 and 0 <= pos < sl):
        return None
    return {"row": i, "request": r, "position": pos, "seq_len": sl, "head": pk % heads}


def _bits(v) -> int:
    return int(np.asarray(v, dtype=f32).reshape(1).view(np.uint32)[0])


@dataclass
class SampleResult:
    j: int
    valid: bool
    row: int = 0
    head: int = 0
    request: int = 0
    position: int = 0
    seq_len: int = 0
    lo: int = 0
    nkeys: int = 0
    bad: bool = False
    finite: bool = True
    judged: bool = False
    z: Optional[np.ndarray] = None      # (D,) scores, NaN -> inf
    zmax: float = 0.0
    dim: int = 0
    ref: Optional[np.ndarray] = None
    bound: Optional[np.ndarray] = None
    write_checked: bool = False
    write_content_bad: bool = False
    write_slot_bad: bool = False


@dataclass
class CheckOut:
    state: np.ndarray                     # int64[COLS] (the input row plus this call)
    capm: np.ndarray                      # int64[CAPM]
    capq: np.ndarray                      # float32[D]
    capo: np.ndarray                      # float32[D]
    samples: list = field(default_factory=list)


def check(q, o, kv, key, val, qsl, seq_lens, bt, slots, *, step: int, active: bool = True, nl: int = 1,
          idx: int = 0, scale: float, left: int = -1, line: float = ATTN_Z, has_write: bool = True,
          dtype: str = "bf16", samples: int = SAMPLES, state=None, capm=None, capq=None, capo=None,
          kernel_keys: bool = False) -> CheckOut:
    """One call of the check: serve_attn.py:165-280 (`attn_check_torch`).

    q, o: (T, Hq, D) float32 (the 16-bit values); kv: (blocks, Hkv, N, 2D) float32; key/val: (T, Hkv, D) float32
    (compared bit for bit as 16-bit words of `dtype`); qsl (R+1,), seq_lens (R,), bt (R, W) ints; slots (SN,) ints.
    state / capm / capq / capo: the layer's rows before the call (zeros if None)."""
    q = np.asarray(q, f32)
    o = np.asarray(o, f32)
    kv = np.asarray(kv, f32)
    T, Hq, D = q.shape
    NB, Hkv, N = kv.shape[0], kv.shape[1], kv.shape[2]
    qsl = np.asarray(qsl, np.int64)
    seq_lens = np.asarray(seq_lens, np.int64)
    bt = np.asarray(bt, np.int64)
    R, W = seq_lens.shape[0], bt.shape[1]
    u, sig_o, hsig_p, g_qk = bound_consts(dtype, D)
    gq = Hq // Hkv
    st = np.zeros(COLS, np.int64) if state is None else np.array(state, np.int64).copy()
    cm = np.zeros(CAPM, np.int64) if capm is None else np.array(capm, np.int64).copy()
    cq = np.zeros(D, f32) if capq is None else np.array(capq, f32).copy()
    co = np.zeros(D, f32) if capo is None else np.array(capo, f32).copy()
    out = CheckOut(st, cm, cq, co)
    step = int(step) & M32
    live = bool(active) and (step % nl) == idx
    st[C_CALLS] += int(live)
    if not live:
        return out
    ntok = min(int(qsl[R]), T)
    t = np.arange(W * N)
    scale32 = f32(scale)
    for j in range(samples):
        h = (step // nl) * PICK_A + j * PICK_B + idx * PICK_C
        if j % 2 == 0:
            pk = h % max(ntok * Hq, 1)
            i = pk // Hq
            have = ntok > 0
        else:
            rreal = _first_at_least(qsl, R, ntok)
            pk = h % max(rreal * Hq, 1)
            i = int(qsl[min(pk // Hq + 1, R)]) - 1
            have = ntok > 0 and rreal > 0
        i = min(max(i, 0), T - 1)
        r = min(max(_first_at_least(qsl, R, i + 1) - 1, 0), R - 1)
        q0, q1 = int(qsl[r]), int(qsl[r + 1])
        sl = int(seq_lens[r])
        qlen = q1 - q0
        pos = sl - qlen + (i - q0)
        valid = have and qlen > 0 and sl > 0 and 0 <= pos < sl and sl <= W * N
        hq = pk % Hq
        hk = hq // gq
        lo = max(pos - left, 0) if left >= 0 else 0
        nkeys = pos - lo + 1
        sr = SampleResult(j, valid, i, hq, r, pos, sl, lo, nkeys)
        out.samples.append(sr)
        if not valid:
            st[C_SKIP] += 1
            continue
        keep = (t >= lo) & (t <= pos)
        blk = bt[r][np.minimum(t // N, W - 1)]
        okb = (blk >= 0) & (blk < NB)
        bad = bool((keep & ~okb).any())
        blk = np.where(okb, blk, 0)
        rows = kv[blk, hk, t % N].astype(f32)                      # (W*N, 2D)
        rows = np.where(keep[:, None], rows, f32(0))
        K, V = rows[:, :D], rows[:, D:2 * D]
        qv = q[i, hq]
        with np.errstate(all="ignore"):
            s = (K @ qv).astype(f32) * scale32
            s = np.where(keep, s, f32(-np.inf))
            m = f32(s.max())
            p = np.where(keep, np.exp(s - m), f32(0)).astype(f32)
            e = (f32(g_qk) * scale32 * (np.abs(K) @ np.abs(qv)).astype(f32) + f32(TWO22) * np.abs(s) +
                 f32(TWO21)).astype(f32)
            pe = np.where(keep, p * e, f32(0)).astype(f32)
            l = f32(p.sum(dtype=f32))
            Va = np.abs(V)
            ref = ((p @ V).astype(f32) / l).astype(f32)
            A = ((p @ Va).astype(f32) / l).astype(f32)
            E = (((pe @ Va).astype(f32) + np.abs(ref) * f32(pe.sum(dtype=f32))) / l).astype(f32)
            Sm = (f32(hsig_p) * np.where(keep[:, None], Va, f32(0)).sum(0, dtype=f32) / l).astype(f32)
            gam = f32((f32(nkeys) / f32(16) + f32(32)) * f32(TWO22) + f32(TWO22) * abs(m))
            bound = ((f32(2 * u) + gam) * (A + np.abs(ref)) + E + Sm + f32(sig_o)).astype(f32)
            ov = o[i, hq]
            z = (np.abs(ov - ref) / bound).astype(f32)
        z = np.where(np.isnan(z) | np.isposinf(z), f32(np.inf), z)
        finite = bool(np.isfinite(ref).all() and np.isfinite(bound).all() and np.isfinite(l) and l > 0)
        judged = (not bad) and finite
        sr.bad, sr.finite, sr.judged, sr.z, sr.ref, sr.bound = bad, finite, judged, z, ref, bound
        dz = int(np.argmax(z))
        zmax = float(z[dz]) if judged else 0.0
        sr.zmax, sr.dim = zmax, dz
        if judged and (zmax > 0 or not kernel_keys):
            zb = _bits(zmax) << 32
            keys = [zb | i, zb | hq, zb | dz, zb | _bits(ov[dz]), zb | _bits(ref[dz]), zb | step, zb | pos]
            for c_, kk in enumerate(keys):
                st[c_] = max(st[c_], kk)
        st[C_SAMPLES] += int(judged)
        st[C_BADBLK] += int(bad)
        st[C_UNJ] += int((not bad) and not finite)
        st[C_KEYS] += nkeys if judged else 0
        if judged and zmax > line and cm[CM_CLAIM] == 0:
            cm[:] = [1, i, hq, r, pos, sl, lo, step, _bits(zmax), 0, dz, hk]
            cq[:] = qv
            co[:] = ov
        if has_write:
            slots_ = np.asarray(slots, np.int64)
            sn = slots_.shape[0]
            ic = min(i, sn - 1)
            s_i = int(slots_[ic])
            want = int(bt[r][min(max(pos // N, 0), W - 1)]) * N + pos % N
            okw = i < sn and 0 <= s_i < NB * N
            if okw:
                cache = kv[s_i // N, :, s_i % N]                       # (Hkv, 2D)
                ck, cv = cache[:, :D], cache[:, D:2 * D]
                mk = _words(ck, dtype) != _words(np.asarray(key, f32)[ic], dtype)
                mv = _words(cv, dtype) != _words(np.asarray(val, f32)[ic], dtype)
                badc = bool(mk.any() or mv.any())
                bads = s_i != want
                sr.write_checked, sr.write_content_bad, sr.write_slot_bad = True, badc, bads
                big = Hkv * D
                flat = np.arange(big).reshape(Hkv, D)
                fk = int(np.where(mk, flat, big).min())
                fv = int(np.where(mv, flat, big).min())
                isv = fk >= big
                first = fv if isv else fk
                where_ = ((first // D) << 12) | ((first % D) << 1) | int(isv)
                kind = (W_CONTENT if badc else 0) | (W_SLOT if bads else 0)
                st[C_WN] += 1
                st[C_WBAD] += int(badc)
                st[C_WSLOT] += int(bads)
                if badc or bads:
                    s31 = (step & S31) << 32
                    st[C_WLAST] = max(st[C_WLAST], s31 | i)
                    st[C_WWHERE] = max(st[C_WWHERE], s31 | (kind << 28) | (where_ if badc else 0))
    return out


def _words(x, dtype: str) -> np.ndarray:
    """16-bit words of fp32 values that are exactly representable in `dtype`."""
    x = np.asarray(x, f32)
    if dtype == "fp16":
        return x.astype(np.float16).view(np.uint16)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def recheck(q_row, o_row, k_rows, v_rows, scale: float, dtype: str, line: float = ATTN_Z) -> dict:
    """serve_attn.py:764-798: the kept sample recomputed in float64 with the same bound."""
    q = np.asarray(q_row, np.float64)
    o = np.asarray(o_row, np.float64)
    K = np.asarray(k_rows, np.float64)
    V = np.asarray(v_rows, np.float64)
    D = q.shape[-1]
    u, sig_o, hsig_p, g_qk = bound_consts(dtype, D)
    s = (K @ q) * scale
    m = s.max()
    p = np.exp(s - m)
    l = p.sum()
    ref = (p @ V) / l
    A = (p @ np.abs(V)) / l
    e = g_qk * scale * (np.abs(K) @ np.abs(q)) + TWO22 * np.abs(s) + TWO21
    E = ((p * e) @ np.abs(V) + np.abs(ref) * (p * e).sum()) / l
    Sm = hsig_p * np.abs(V).sum(0) / l
    gam = (K.shape[0] / 16 + 32) * TWO22 + TWO22 * abs(float(m))
    bound = (2 * u + gam) * (A + np.abs(ref)) + E + Sm + sig_o
    with np.errstate(all="ignore"):
        z = np.abs(o - ref) / bound
    z = np.where(np.isnan(z) | np.isposinf(z), np.inf, z)
    worst = float(z.max()) if z.size else 0.0
    bad = int((z > line).sum())
    out = {"worst_score": worst, "outputs_over_line": bad, "outputs": int(o.size), "keys": int(K.shape[0])}
    if not np.isfinite(ref).all():
        return {**out, "verdict": "not_judged"}
    if z.size:
        d = int(np.argmax(z))
        out.update(dim=d, output=float(o[d]), expected=float(ref[d]))
    return {**out, "verdict": "output_wrong" if bad else "output_agrees"}
