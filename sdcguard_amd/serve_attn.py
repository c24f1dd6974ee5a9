"""Sampled attention recompute from a paged KV cache, and the check of the sampled tokens' own KV writes.

The check of serve_attn.py (reference): at a checked call, SAMPLES (token, head) outputs of one attention layer are
recomputed in fp32 from the query row and the request's keys and values, read from the paged KV cache through the
block table (block bt[r, t // block_size], slot t % block_size), and scored against the first-order rounding bound
of a correct FlashAttention / Triton backend (serve_attn.py:14-36); the sampled token's own KV write is compared bit
for bit with the cache slot the block table gives its position.  The GPU work is one launch of the library's
`sdc_attn_check` (csrc/attn_check.hip); there is no CPU implementation of the check.

Kept as in the reference, because they are its state format and its sample choice: the constants below, the
18-column state row and its column order, the 12-column capture row, the packed keys (score bits << 32 | value),
and the sample-picking rule (sample_python).
"""
from __future__ import annotations

import bisect
import ctypes
import math
from typing import Optional

import torch

from . import _lib

ATTN_Z = 4.0              # the line (serve_attn.py:73)
MIN_LINE = 1.5
SAMPLES = 4               # (token, head) pairs per checked call
CAP_ROWS = 65536          # most keys and values kept for an alarming sample
LOG_R = 17
MAX_REQUESTS = (1 << (LOG_R - 1)) - 1
M32 = 0xFFFFFFFF
S31 = 0x7FFFFFFF
PICK_A, PICK_B, PICK_C = 1000003, 7919, 104729
TWO22, TWO21, TWO23 = 2.0 ** -22, 2.0 ** -21, 2.0 ** -23
COLS = 18
(C_ZT, C_ZH, C_ZD, C_ZO, C_ZR, C_ZS, C_ZP, C_CALLS, C_SAMPLES, C_SKIP, C_UNJ, C_BADBLK, C_KEYS, C_WN, C_WBAD,
 C_WSLOT, C_WLAST, C_WWHERE) = range(COLS)
CAPM = 12
CM_CLAIM, CM_ROW, CM_HEAD, CM_REQ, CM_POS, CM_SL, CM_LO, CM_STEP, CM_Z, CM_KEPT, CM_DIM, CM_HK = range(CAPM)
W_CONTENT, W_SLOT = 1, 2


def f32_of_bits(bits: int) -> float:
    return float(torch.tensor([int(bits) & M32], dtype=torch.int64).to(torch.int32).view(torch.float32).item())


def dtype_consts(dtype: torch.dtype) -> tuple:
    """(unit roundoff, output spacing) of the outputs' dtype (serve_norm.py:69-77)."""
    if dtype == torch.float16:
        return 2.0 ** -11, 2.0 ** -24
    return 2.0 ** -8, 1e-37


def p_spacing(dtype: torch.dtype) -> float:
    """Half the subnormal spacing of P's dtype, or fp32's smallest normal (serve_attn.py:106-109)."""
    return 2.0 ** -25 if dtype == torch.float16 else 2.0 ** -126


def bound_consts(dtype: torch.dtype, head_size: int) -> tuple:
    """(u, output spacing, P spacing, q.k accumulation coefficient) for outputs in dtype (serve_attn.py:115-118)."""
    u, sp = dtype_consts(dtype)
    return u, sp, p_spacing(dtype), (head_size + 8) * TWO23


def sample_python(step: int, idx: int, nl: int, j: int, qsl: list, seq_lens: list, rows: int,
                  heads: int) -> Optional[dict]:
    """The (token row, request, position, seq_len, query head) sample j of layer idx of nl takes at a step, or None
    (serve_attn.py:130-157; the kernel takes the same)."""
    nreq = len(seq_lens)
    ntok = min(int(qsl[nreq]), rows)
    if ntok <= 0:
        return None
    h = (step // nl) * PICK_A + j * PICK_B + idx * PICK_C
    if j % 2 == 0:
        pk = h % (ntok * heads)
        i = pk // heads
    else:
        nreal = bisect.bisect_left(qsl, ntok, 0, nreq + 1)      # requests that hold a token of the step
        if nreal <= 0:
            return None
        pk = h % (nreal * heads)
        i = int(qsl[pk // heads + 1]) - 1
    r = bisect.bisect_left(qsl, i + 1, 0, nreq + 1) - 1
    q0, q1, sl = int(qsl[r]), int(qsl[r + 1]), int(seq_lens[r])
    pos = sl - (q1 - q0) + (i - q0)
    if not (0 <= i < rows and q1 > q0 and sl > 0 and 0 <= pos < sl):
        return None
    return {"row": i, "request": r, "position": pos, "seq_len": sl, "head": pk % heads}


def _pow2(x: int) -> int:
    return 1 << (max(1, int(x)) - 1).bit_length()


def workspace_bytes(samples: int, max_keys: int, head_size: int) -> int:
    return int(_lib.lib().sdc_attn_check_workspace(samples, max_keys, head_size))


def buffers(device, slots: int, width: int, cap_rows: int, kv_dtype, samples: int = SAMPLES) -> dict:
    """The buffers the checks of `slots` layers write on one device, allocated once (fixed addresses, so calls can
    be captured in HIP graphs); the workspace is sized for any context length (serve_attn.py:667-678)."""
    bd = _pow2(width)
    ws = workspace_bytes(samples, 1 << 40, width)
    return {"state": torch.zeros(slots, COLS, dtype=torch.int64, device=device),
            "capm": torch.zeros(slots, CAPM, dtype=torch.int32, device=device),
            "capq": torch.zeros(slots, bd, dtype=torch.float32, device=device),
            "capo": torch.zeros(slots, bd, dtype=torch.float32, device=device),
            "capkv": torch.zeros(max(1, cap_rows), 2, bd, dtype=kv_dtype, device=device),
            "capkvm": torch.zeros(4, dtype=torch.int32, device=device),
            "ws": torch.zeros(max(ws, 1), dtype=torch.uint8, device=device),
            "ctrl": torch.zeros(2, dtype=torch.int64, device=device),
            "samples": samples}


def _index32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def _call_args(q, o, kv, key, val, qsl, seq_lens, bt, slots, state, slot, ctrl, nl, idx, scale, left, line, capm,
               capq, capo, capkv, capkvm, has_write, keep_kv, samples):
    """The C-ABI arguments of one check, up to and including `samples` (sdc_attn_check's order), and the flags."""
    _lib.require_gpu(q, o, kv, state)
    T, Hq, D = q.shape
    NB, Hkv, N = kv.shape[0], kv.shape[1], kv.shape[2]
    R, W = seq_lens.shape[0], bt.shape[1]
    if q.stride(-1) != 1 or o.stride(-1) != 1 or o.shape != q.shape:
        raise ValueError("q and o must be [T, Hq, D] with the last dimension contiguous")
    if kv.shape[3] != 2 * D or kv.dtype != q.dtype or o.dtype != q.dtype:
        raise ValueError("a KV cache layout the check does not read: [blocks, Hkv, block_size, 2 * head_size] in "
                         "the queries' dtype")
    if R > MAX_REQUESTS:
        raise ValueError(f"{R} requests in a step: the kernel takes at most {MAX_REQUESTS}")
    if not 0 <= int(slot) < state.shape[0] or state.shape[1] != COLS or ctrl.numel() < 2:
        raise ValueError("slot outside the state rows, or buffers not made by buffers()")
    if capm is not None and (capm.shape[0] <= int(slot) or capm.shape[1] != CAPM or capq.shape[0] <= int(slot) or
                             capo.shape != capq.shape or capq.shape[1] < D):
        raise ValueError("capture buffers too small for this slot or head size")
    if capkv is not None and (capkv.dim() != 3 or capkv.shape[1] != 2 or
                              (capq is not None and capkv.shape[2] != capq.shape[1])):
        raise ValueError("capkv must be [rows, 2, width] with the width of capq")
    qsl, seq_lens, bt = _index32(qsl), _index32(seq_lens), _index32(bt)
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    if has_write:
        if key.stride(-1) != 1 or val.stride(-1) != 1:
            raise ValueError("key and val must have a contiguous last dimension")
        if slots.dtype != torch.int64:
            slots = slots.to(torch.int64)
        kk, vv, sl_ = key, val, slots
    else:
        kk, vv, sl_ = None, None, None
    keep = bool(keep_kv) and capkv is not None and capkv.dtype == kv.dtype and capkv.shape[-1] >= D
    cap_rows = capkv.shape[0] if keep else 0
    args = (_lib.dtype_code(q.dtype), q.data_ptr(), q.stride(0), q.stride(1), o.data_ptr(), o.stride(0), o.stride(1),
            T, Hq, D, kv.data_ptr(), kv.stride(0), kv.stride(1), kv.stride(2), kv.stride(3), NB, Hkv, N,
            _lib.ptr(kk), kk.stride(0) if kk is not None else 0, kk.stride(1) if kk is not None else 0,
            _lib.ptr(vv), vv.stride(0) if vv is not None else 0, vv.stride(1) if vv is not None else 0,
            qsl.data_ptr(), seq_lens.data_ptr(), R, bt.data_ptr(), bt.stride(0), W,
            _lib.ptr(sl_), sl_.shape[0] if sl_ is not None else 0,
            state.data_ptr(), int(slot), ctrl.data_ptr(), int(nl), int(idx), float(scale), int(left), float(line),
            _lib.ptr(capm), _lib.ptr(capq), _lib.ptr(capo), capq.shape[1] if capq is not None else 0,
            _lib.ptr(capkv) if keep else None, _lib.ptr(capkvm) if keep else None, cap_rows, int(samples))
    # the index tensors converted above must live until the kernel has read them: the caller's stream orders them
    return args, (1 if has_write else 0), (1 if keep else 0), (qsl, seq_lens, bt, sl_)


def attn_check(q, o, kv, key, val, qsl, seq_lens, bt, slots, state, slot, ctrl, nl, idx, scale, left, line, capm,
               capq, capo, capkv, capkvm, ws, has_write, keep_kv, samples: int = SAMPLES,
               scores_out: Optional[torch.Tensor] = None) -> None:
    """One check of a call (serve_attn.attn_check_triton's arguments): q, o [T, Hq, D], kv [blocks, Hkv, N, 2D],
    key / val [T, Hkv, D], vLLM's query_start_loc, seq_lens, block_table and slot_mapping; state, capm, capq, capo,
    capkv, capkvm, ws and ctrl from buffers().  Queues one kernel on the current stream; never synchronises."""
    args, hw, keep, _held = _call_args(q, o, kv, key, val, qsl, seq_lens, bt, slots, state, slot, ctrl, nl, idx,
                                       scale, left, line, capm, capq, capo, capkv, capkvm, has_write, keep_kv,
                                       samples)
    rc = _lib.lib().sdc_attn_check(*args, _lib.ptr(ws), ws.numel() * ws.element_size() if ws is not None else 0,
                                   hw, keep, _lib.ptr(scores_out), _lib.stream_of(q))
    _lib.check(rc, "sdc_attn_check")


SCRATCH_BYTES = 4456448      # the static workspace of attn_check_noalloc on each GPU (SDC_ATTN_SCRATCH_BYTES)


def attn_check_noalloc(q, o, kv, key, val, qsl, seq_lens, bt, slots, state, slot, ctrl, nl, idx, scale, left, line,
                       capm, capq, capo, capkv, capkvm, has_write, keep_kv, samples: int = SAMPLES,
                       scores_out: Optional[torch.Tensor] = None) -> None:
    """attn_check without a workspace: the library uses a static device array of SCRATCH_BYTES on q's GPU, so the
    call allocates nothing (for graph capture and serving loops that cannot allocate).  Calls that overlap in time
    on one GPU share that array and must not be made."""
    with torch.cuda.device(q.device):
        args, hw, keep, _held = _call_args(q, o, kv, key, val, qsl, seq_lens, bt, slots, state, slot, ctrl, nl, idx,
                                           scale, left, line, capm, capq, capo, capkv, capkvm, has_write, keep_kv,
                                           samples)
        rc = _lib.lib().sdc_attn_check_noalloc(*args, hw, keep, _lib.ptr(scores_out), _lib.stream_of(q))
    if rc == _lib.SDC_EWORKSPACE:
        raise _lib.HipLibraryError(f"sdc_attn_check_noalloc: the call needs more than the {SCRATCH_BYTES} bytes of "
                                   "static workspace (use attn_check with a workspace)")
    _lib.check(rc, "sdc_attn_check_noalloc")


attn_check_triton = attn_check     # the reference's name for the device check


def run_case(c: dict, b: dict, *, step=0, nl=1, idx=0, slot=0, line=ATTN_Z, left=-1, has_write=True,
             keep_kv=True, active=True, scores_out=None) -> None:
    """One check of the call c (make_case) with the buffers b (buffers), at a step (serve_attn.py:681-690)."""
    b["ctrl"][0] = step
    b["ctrl"][1] = 1 if active else 0
    attn_check(c["q"], c["o"], c["kv"], c["key"], c["val"], c["qsl"], c["seq_lens"], c["bt"], c["slots"],
               b["state"], slot, b["ctrl"], nl, idx, c["scale"], left, line, b["capm"], b["capq"], b["capo"],
               b["capkv"], b["capkvm"], b["ws"], has_write, keep_kv, samples=b.get("samples", SAMPLES),
               scores_out=scores_out)


def make_case(device, dtype, *, D=64, Hq=4, Hkv=2, N=16, NB=12, lens=((5, 1), (37, 9), (0, 0)), seed=0,
              padded_rows=3) -> dict:
    """A small paged-attention call with the outputs of a correct backend (float64 attention rounded to dtype):
    requests (seq_len, query_len), (0, 0) a graph-padding request, padded_rows rows past the real tokens; block
    ids drawn without repeats (serve_attn.py:621-664 builds the same kind of call)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    R = len(lens)
    qlens = [ql for _, ql in lens]
    T = sum(qlens) + padded_rows
    W = max(1, max(-(-sl // N) for sl, _ in lens))
    order = torch.randperm(NB, generator=g)
    bt = torch.zeros(R, W, dtype=torch.int32)
    used = 0
    for r, (sl, _) in enumerate(lens):
        nblk = -(-sl // N)
        bt[r, :nblk] = order[(torch.arange(nblk) + used) % NB].to(torch.int32)
        used += nblk
    kv = (torch.randn(NB, Hkv, N, 2 * D, generator=g) * 0.8).to(dtype)
    q = (torch.randn(T, Hq, D, generator=g) * 0.5).to(dtype)
    qsl = torch.zeros(R + 1, dtype=torch.int32)
    qsl[1:] = torch.tensor(qlens, dtype=torch.int32).cumsum(0)
    sls = torch.tensor([sl for sl, _ in lens], dtype=torch.int32)
    slots = torch.full((T,), -1, dtype=torch.int64)
    key = torch.zeros(T, Hkv, D, dtype=dtype)
    val = torch.zeros(T, Hkv, D, dtype=dtype)
    o = torch.zeros(T, Hq, D, dtype=dtype)
    kv64 = kv.double()
    for r, (sl, ql) in enumerate(lens):
        if ql == 0:
            continue
        t = torch.arange(sl)
        rows = kv64[bt[r, t // N].long(), :, t % N]                 # [sl, Hkv, 2D]
        for jj in range(ql):
            i = int(qsl[r]) + jj
            pos = sl - ql + jj
            blk, off = int(bt[r, pos // N]), pos % N
            slots[i] = blk * N + off
            key[i] = kv[blk, :, off, :D]
            val[i] = kv[blk, :, off, D:]
            ks = rows[:pos + 1]                                      # [pos+1, Hkv, 2D]
            for hq in range(Hq):
                hk = hq // (Hq // Hkv)
                s = ks[:, hk, :D] @ q[i, hq].double() * D ** -0.5
                o[i, hq] = (torch.softmax(s, 0) @ ks[:, hk, D:]).to(dtype)
    return {"q": q.to(device), "o": o.to(device), "kv": kv.to(device), "key": key.to(device), "val": val.to(device),
            "qsl": qsl.to(device), "seq_lens": sls.to(device), "bt": bt.to(device), "slots": slots.to(device),
            "scale": D ** -0.5}


def recheck(q_row: torch.Tensor, o_row: torch.Tensor, k_rows: torch.Tensor, v_rows: torch.Tensor, scale: float,
            dtype: torch.dtype, line: float = ATTN_Z) -> dict:
    """An alarming sample's recompute in float64 from the keys and values it attended (kept exactly by the check),
    with the same bound: the host-side confirmation an alert carries (serve_attn.py:764-798).  It runs on the
    captured rows after the read-back, not in the check."""
    D = q_row.shape[-1]
    q, o = q_row.double().cpu(), o_row.double().cpu()
    K, V = k_rows.double().cpu(), v_rows.double().cpu()
    u, sig_o, hsig_p, g_qk = bound_consts(dtype, D)
    s = (K @ q) * scale
    mx = s.max()
    p = torch.exp(s - mx)
    tot = p.sum()
    ref = (p @ V) / tot
    Va = V.abs()
    e = g_qk * scale * (K.abs() @ q.abs()) + TWO22 * s.abs() + TWO21
    bound = (2 * u + (K.shape[0] / 16 + 32) * TWO22 + TWO22 * abs(float(mx))) * ((p @ Va) / tot + ref.abs()) + \
        ((p * e) @ Va + ref.abs() * (p * e).sum()) / tot + hsig_p * Va.sum(0) / tot + sig_o
    z = torch.nan_to_num((o - ref).abs() / bound, nan=math.inf, posinf=math.inf)
    worst = float(z.max()) if z.numel() else 0.0
    over = int((z > line).sum())
    out = {"worst_score": worst, "outputs_over_line": over, "outputs": int(o.numel()), "keys": int(K.shape[0])}
    if not torch.isfinite(ref).all():
        return {**out, "verdict": "not_judged", "why": "the kept keys or values are not finite"}
    if z.numel():
        d = int(z.argmax())
        out.update(dim=d, output=float(o[d]), expected=float(ref[d]))
    if over:
        return {**out, "verdict": "output_wrong",
                "why": f"{over} of {o.numel()} values of the kept output are more than {line:g} times the rounding "
                       "bound from attention recomputed in float64 from its query and the keys and values it "
                       "attended"}
    return {**out, "verdict": "output_agrees",
            "why": "the float64 recompute of the kept sample agrees with its output: the GPU's check disagreed"}


def decode_state(row) -> dict:
    """The 18-column state row of one layer as a dict (the reference's AttnChecks._report reads the same)."""
    k = [int(v) for v in (row.tolist() if hasattr(row, "tolist") else row)]
    return {"max_z": f32_of_bits(k[C_ZT] >> 32), "row": k[C_ZT] & M32, "head": k[C_ZH] & M32,
            "dim": k[C_ZD] & M32, "output": f32_of_bits(k[C_ZO]), "expected": f32_of_bits(k[C_ZR]),
            "step": k[C_ZS] & M32, "position": k[C_ZP] & M32, "calls": k[C_CALLS], "samples": k[C_SAMPLES],
            "skipped": k[C_SKIP], "unjudged": k[C_UNJ], "bad_blocks": k[C_BADBLK], "keys": k[C_KEYS],
            "writes_checked": k[C_WN], "writes_wrong": k[C_WBAD], "slots_wrong": k[C_WSLOT],
            "write_last": k[C_WLAST], "write_where": k[C_WWHERE]}


# ------------------------------------------------------------------------------------------ the serving layers
# Which attention layers the check models (the reference's why_not / call_issue, serve_attn.py:800-880, read the
# same attributes of the serving stack's layer and backend): one ordered rule table per layer, and the per-call
# conditions read from the call's tensors and metadata on the host.
BACKENDS = ("FlashAttentionImpl", "TritonAttentionImpl")


def _window_of(impl) -> tuple:
    sw = getattr(impl, "sliding_window", (-1, -1))
    return tuple(sw) if sw is not None else (-1, -1)


def _heads(impl) -> tuple:
    return tuple(getattr(impl, a, None) for a in ("head_size", "num_heads", "num_kv_heads"))


_LAYER_RULES = (
    (lambda layer, impl: type(layer).__name__ == "Attention",
     lambda layer, impl: f"{type(layer).__name__}: only plain decoder attention layers are checked"),
    (lambda layer, impl: type(impl).__name__ in BACKENDS,
     lambda layer, impl: f"{type(impl).__name__}: only the FlashAttention and Triton backends' rounding is modelled"),
    (lambda layer, impl: not (type(impl).__name__ == "FlashAttentionImpl" and
                              getattr(impl, "vllm_flash_attn_version", None) not in (None, 2, 3)),
     lambda layer, impl: f"FlashAttention {getattr(impl, 'vllm_flash_attn_version', None)} (the bound is written for "
                         "versions 2 and 3)"),
    (lambda layer, impl: str(getattr(impl, "attn_type", "decoder")).lower().endswith("decoder") and
     "encoder" not in str(getattr(impl, "attn_type", "decoder")).lower(),
     lambda layer, impl: f"attention type {getattr(impl, 'attn_type', None)}"),
    (lambda layer, impl: getattr(impl, "alibi_slopes", None) is None and not getattr(impl, "use_alibi_sqrt", False),
     lambda layer, impl: "ALiBi"),
    (lambda layer, impl: getattr(impl, "sinks", None) is None, lambda layer, impl: "attention sinks"),
    (lambda layer, impl: getattr(impl, "logits_soft_cap", 0) in (0, None, 0.0), lambda layer, impl: "a logit soft cap"),
    (lambda layer, impl: _window_of(impl) == (-1, -1), lambda layer, impl: "a sliding window"),
    (lambda layer, impl: getattr(impl, "chunk_lookback", -1) in (-1, None),
     lambda layer, impl: "chunked local attention"),
    (lambda layer, impl: (getattr(impl, "dcp_world_size", 1) or 1) <= 1,
     lambda layer, impl: "decode context parallelism"),
    (lambda layer, impl: str(getattr(impl, "kv_cache_dtype", "auto")) in ("auto", "bfloat16", "float16"),
     lambda layer, impl: f"KV cache dtype {getattr(impl, 'kv_cache_dtype', None)}"),
    (lambda layer, impl: all(isinstance(v, int) and v > 0 for v in _heads(impl)) and
     _heads(impl)[1] % _heads(impl)[2] == 0,
     lambda layer, impl: "head counts it can't read"),
    (lambda layer, impl: _heads(impl)[0] <= 256, lambda layer, impl: f"head size {_heads(impl)[0]}"),
    (lambda layer, impl: getattr(layer, "head_size_v", _heads(impl)[0]) == _heads(impl)[0],
     lambda layer, impl: "values of another size than the keys"),
)


def why_not(layer, impl, model_dtype=None) -> Optional[str]:
    """Why an attention layer of the serving stack is not checked, or None."""
    for holds, why in _LAYER_RULES:
        if not holds(layer, impl):
            return why(layer, impl)
    kvd = str(getattr(impl, "kv_cache_dtype", "auto"))
    if model_dtype is not None and kvd != "auto" and kvd != str(model_dtype).replace("torch.", ""):
        return f"KV cache dtype {kvd} differs from the model's"
    return None


def call_issue(impl, query, output, kv_cache, md, output_scale=None) -> Optional[str]:
    """Why one call is not checked (shapes and the metadata's host fields), or None."""
    if output_scale is not None:
        return "fused output quantization"
    if not all(isinstance(t, torch.Tensor) for t in (query, output, kv_cache)):
        return "inputs it can't read"
    if query.dim() != 3 or output.dim() != 3 or kv_cache.dim() != 4:
        return "tensor layouts it doesn't know"
    D = query.shape[2]
    if output.shape != query.shape or output.dtype not in (torch.bfloat16, torch.float16) or \
            query.dtype != output.dtype or output.stride(-1) != 1 or query.stride(-1) != 1:
        return "outputs it can't compare"
    if kv_cache.dtype != query.dtype or kv_cache.shape[1] != impl.num_kv_heads or kv_cache.shape[3] != 2 * D:
        return "a KV cache layout it doesn't know"
    if getattr(md, "causal", True) is not True:
        return "attention that isn't causal for every request"
    if any(getattr(md, f, None) is not None for f in ("mm_prefix_query_range_tensor", "mm_prefix_range_tensor",
                                                      "rswa_prefix_lens")):
        return "multimodal prefix ranges or R-SWA"
    for f in ("query_start_loc", "seq_lens", "block_table"):
        if not isinstance(getattr(md, f, None), torch.Tensor):
            return f"metadata without {f}"
    if md.block_table.dim() != 2 or md.query_start_loc.shape[0] != md.seq_lens.shape[0] + 1 or \
            md.block_table.shape[0] < md.seq_lens.shape[0]:
        return "metadata it can't read"
    if md.seq_lens.shape[0] > MAX_REQUESTS:
        return f"more than {MAX_REQUESTS:,} requests in a step"
    return None


from .stepchecks import W_STEP, Binding, Registered, StepChecks  # noqa: E402  (after the kernel wrappers)


class AttnChecks(StepChecks):
    """The attention layers one serving guard checks (ServeGuard.attn_checks()).  add() each layer, finalize() once
    before any graph is captured (it numbers the layers' turns -- at step s the layer with index s % layers
    recomputes its samples -- sizes the kept-keys buffer and gives each layer its binding, layer._sdcguard_attn),
    check() after each call of a layer's backend, mark_step() / end_step() around each model step, poll() to read.
    The state rows are the kernel's 18 columns (serve_attn.py:86-92)."""

    DETECTOR = "serve_attn"
    COLS = COLS
    CAPTURE = {"meta": torch.int32, "q": torch.float32, "o": torch.float32}
    READ_CAPTURE = ("meta",)

    def __init__(self, guard=None, line: float = ATTN_Z):
        line = float(line)
        if not MIN_LINE <= line < float("inf"):
            raise ValueError(f"the attention check's line must be at least {MIN_LINE} (a correct output scores at "
                             f"most 1), not {line!r}")
        super().__init__(guard)
        self.line = line
        self.finalized = False
        self.shared: dict = {}                 # device -> {"capkv", "capkvm", "ws"}: one kept sample per device
        self.cap_rows = 0
        self.not_checked_calls: dict = {}      # why -> calls (seen on the host)
        self.worst_seen: dict = {}
        self.calls_seen: dict = {}
        self.stats.update(calls_checked=0, samples=0, skipped=0, unjudged=0, keys=0, bad_blocks=0,
                          writes_checked=0, writes_wrong=0, slots_wrong=0, graph_calls=0)
        self._in_step = False                  # between mark_step and end_step (the host's view, for eager calls)

    def add(self, layer, impl, name: str, device, model_dtype=None) -> Optional[int]:
        if self.finalized:
            raise RuntimeError("attention layers are added before finalize()")
        why = why_not(layer, impl, model_dtype)
        if why is None and getattr(layer, "_sdcguard_attn", None) is not None:
            why = "already checked by another ServeGuard"
        if why is None and torch.device(device).type != "cuda":
            why = "not on a GPU"
        if why:
            self._refuse(name, why)
            return None
        D, Hq, Hkv = _heads(impl)
        width = _pow2(D)
        b = self._register(name, layer, device, widths={"meta": CAPM, "q": width, "o": width}, impl=impl,
                           scale=float(impl.scale), left=int(_window_of(impl)[0]), D=D, Hq=Hq, Hkv=Hkv,
                           write=getattr(impl, "kv_sharing_target_layer_name", None) is None,
                           backend=type(impl).__name__)
        return b.slot

    def finalize(self, max_len: int = 32768, kv_dtype=torch.bfloat16) -> int:
        """Number the layers' turns, allocate the per-device buffers (the kept sample's keys and values: up to
        min(max_len, CAP_ROWS) rows) and bind the layers.  Before any graph is captured."""
        if self.finalized:
            return len(self.layers)
        self.cap_rows = min(int(max_len), CAP_ROWS)
        per_dev: dict = {}
        for lay in self.layers:
            per_dev.setdefault(lay.device, []).append(lay)
        for dev, lays in per_dev.items():
            for turn, lay in enumerate(lays):
                lay.info["index"], lay.info["count"] = turn, len(lays)
            width = max(_pow2(lay.info["D"]) for lay in lays)
            ws = workspace_bytes(SAMPLES, 1 << 40, width)
            with torch.inference_mode(False):
                self.shared[dev] = {"capkv": torch.zeros(max(1, self.cap_rows), 2, width, dtype=kv_dtype,
                                                         device=dev),
                                    "capkvm": torch.zeros(4, dtype=torch.int32, device=dev),
                                    "ws": torch.zeros(max(ws, 1), dtype=torch.uint8, device=dev)}
        for n, lay in enumerate(self.layers):
            lay.module._sdcguard_attn = Binding(self, n)
        self.finalized = True
        return len(self.layers)

    def _skip(self, why: str) -> None:
        self.not_checked_calls[why] = self.not_checked_calls.get(why, 0) + 1

    def check(self, binding: Binding, impl, query, key, value, kv_cache, md, output, output_scale=None) -> None:
        """After one call of a registered layer's backend.  Inside a graph capture the kernel is always queued (the
        step's layer is chosen on the device from the step word); in eager calls during a marked step only the
        step's layer queues it; outside marked steps (warm-up runs) every layer does, and the kernel returns at once
        (it is compiled ahead of time: nothing is built during a capture)."""
        lay = binding.layer
        dev = lay.device
        if torch.compiler.is_compiling():
            return self._skip("traced by torch.compile")
        capturing = torch.cuda.is_current_stream_capturing()
        if capturing:
            self.stats["graph_calls"] += 1
        elif self._in_step and self.marked % lay.info["count"] != lay.info["index"]:
            return None
        why = call_issue(impl, query, output, kv_cache, md, output_scale)
        if why:
            return self._skip(why)
        T = min(int(query.shape[0]), int(getattr(md, "num_actual_tokens", query.shape[0]) or query.shape[0]))
        if T <= 0:
            return None
        has_write = bool(lay.info["write"]) and all(isinstance(t, torch.Tensor) for t in (key, value)) and \
            isinstance(getattr(md, "slot_mapping", None), torch.Tensor) and key.dim() == 3 and value.dim() == 3 and \
            key.dtype == kv_cache.dtype and value.dtype == kv_cache.dtype and key.stride(-1) == 1 and \
            value.stride(-1) == 1 and key.shape[0] == query.shape[0] and value.shape[0] == query.shape[0]
        tab, sh = self.tables[dev], self.shared[dev]
        c = tab.capture
        with torch.no_grad(), torch.autocast(device_type="cuda", enabled=False):
            attn_check(query[:T], output[:T], kv_cache, key if has_write else None, value if has_write else None,
                       md.query_start_loc, md.seq_lens, md.block_table, md.slot_mapping if has_write else None,
                       tab.state, lay.slot, tab.word.view(W_STEP, 2), lay.info["count"], lay.info["index"],
                       lay.info["scale"], lay.info["left"], self.line, c["meta"], c["q"], c["o"], sh["capkv"],
                       sh["capkvm"], sh["ws"], has_write, self.cap_rows > 0)
        lay.info["dtype"] = output.dtype

    def mark_step(self, step: int, rows: Optional[int] = None) -> None:
        super().mark_step(step, rows)
        self._in_step = True

    def end_step(self) -> None:
        super().end_step()
        self._in_step = False

    def detach(self) -> None:
        super().detach()
        self.shared.clear()
        self.finalized = False

    def _unbind(self, lay: Registered) -> None:
        lay.module.__dict__.pop("_sdcguard_attn", None)

    def coverage(self) -> dict:
        out = super().coverage()
        out.update(calls_checked=self.stats["calls_checked"], samples_per_call=SAMPLES, one_layer_a_step=True,
                   calls_not_checked=dict(self.not_checked_calls), samples=self.stats["samples"],
                   keys_recomputed=self.stats["keys"], samples_without_a_token=self.stats["skipped"],
                   samples_not_judged=self.stats["unjudged"], writes_checked=self.stats["writes_checked"])
        return out

    def _count(self, lay: Registered, k: list) -> None:
        lay.calls += k[C_CALLS]
        self.calls_seen[lay.name] = self.calls_seen.get(lay.name, 0) + k[C_CALLS]
        for stat, col in (("calls_checked", C_CALLS), ("samples", C_SAMPLES), ("skipped", C_SKIP),
                          ("unjudged", C_UNJ), ("keys", C_KEYS), ("bad_blocks", C_BADBLK),
                          ("writes_checked", C_WN), ("writes_wrong", C_WBAD), ("slots_wrong", C_WSLOT)):
            self.stats[stat] += k[col]

    def _judged(self, k: list) -> bool:
        return k[C_CALLS] > 0

    def _judge(self, lay: Registered, k: list, captured: dict, window) -> list:
        out = []
        z = f32_of_bits(k[C_ZT] >> 32)
        self.worst_seen[lay.name] = max(self.worst_seen.get(lay.name, 0.0), z)
        lay.worst = max(lay.worst, z)
        if z > self.line:
            meta = [int(v) for v in captured["meta"].tolist()] if "meta" in captured else [0] * CAPM
            out.append(self._output_event(lay, k, meta, window, z))
        if k[C_WBAD] or k[C_WSLOT]:
            out.append(self._write_event(lay, k, window))
        if k[C_BADBLK]:
            out.append(self.emit(lay, float("inf"), None, {
                "where": lay.name, "kind": "attention", "finding": "block_table_out_of_range",
                "samples": k[C_BADBLK], "read_window_steps": window,
                "reading": "a sampled request's block table named KV-cache blocks outside the cache: the attention "
                           "kernel read memory that is not part of the KV cache"}))
        return out

    def _kept_sample(self, lay: Registered, meta: list) -> tuple:
        """(what the kept record says, the float64 recheck of it or None) -- the kept keys and values are read from
        the device and its claim released."""
        if not meta[CM_CLAIM]:
            return None, None
        tab, sh = self.tables[lay.device], self.shared[lay.device]
        D = lay.info["D"]
        q_row, o_row = tab.capture["q"][lay.slot, :D].cpu(), tab.capture["o"][lay.slot, :D].cpu()
        kvm = [int(v) for v in sh["capkvm"].tolist()]
        kept = bool(meta[CM_KEPT]) and kvm[0] == 1 and kvm[1] == lay.slot and kvm[3] == meta[CM_STEP]
        rec = {"row": meta[CM_ROW] & M32, "head": meta[CM_HEAD], "kv_head": meta[CM_HK],
               "request_index": meta[CM_REQ], "position": meta[CM_POS], "seq_len": meta[CM_SL],
               "first_key": meta[CM_LO], "step": (meta[CM_STEP] & M32) if self.marked is not None else None,
               "score": f32_of_bits(meta[CM_Z]), "keys_kept": kept}
        verdict = None
        if kept:
            rows = sh["capkv"][:kvm[2]].cpu()
            verdict = recheck(q_row, o_row, rows[:, 0, :D], rows[:, 1, :D], lay.info["scale"],
                              lay.info.get("dtype", torch.bfloat16), self.line)
            sh["capkvm"].zero_()
        else:
            verdict = {"verdict": "not_rechecked",
                       "why": "the keys and values it attended were not kept (another layer's alert took the "
                              "buffer, or there were more than it holds)"}
        tab.capture["meta"][lay.slot].zero_()
        return rec, verdict

    def _output_event(self, lay: Registered, k: list, meta: list, window, z: float) -> object:
        rec, verdict = self._kept_sample(lay, meta)
        place = {"row": k[C_ZT] & M32, "head": k[C_ZH] & M32, "dim": k[C_ZD] & M32, "position": k[C_ZP] & M32,
                 "step": (k[C_ZS] & M32) if self.marked is not None else None, "output": f32_of_bits(k[C_ZO]),
                 "expected": f32_of_bits(k[C_ZR]), "place": "the read's score maxima"}
        if rec is not None and verdict and verdict.get("outputs_over_line") and verdict.get("dim") is not None:
            place = {"row": rec["row"], "head": rec["head"], "dim": verdict["dim"], "position": rec["position"],
                     "step": rec["step"], "output": verdict["output"], "expected": verdict["expected"],
                     "place": "the kept sample's worst output, rechecked"}
        dtype = lay.info.get("dtype", torch.bfloat16)
        detail = {"where": lay.name, "kind": "attention", "backend": lay.info["backend"],
                  "finding": "output_wrong_or_misread", "max_z": z, **place, "captured": rec,
                  "recheck": verdict or {"verdict": "not_rechecked",
                                         "why": "no sample was kept for this alert (an earlier alert's kept sample "
                                                "has not been read yet)"},
                  "read_window_steps": window, "last_clean_read_steps": self.last_clean(lay.name),
                  "check_config": {"line": self.line, "unit_roundoff": dtype_consts(dtype)[0], "samples": SAMPLES},
                  "reading": "an attention output is farther from attention recomputed from the request's own keys "
                             "and values in the KV cache than a correct backend's rounding allows: wrong arithmetic "
                             "in the attention kernel, or it read other keys than the metadata names"}
        return self.emit(lay, z, place["row"], detail)

    def _write_event(self, lay: Registered, k: list, window) -> object:
        last, wh = k[C_WLAST], k[C_WWHERE]
        kind, info = (wh >> 28) & 0xF, wh & 0x0FFFFFFF
        from .serve_fp8 import unwrap31
        latest = {"step": unwrap31(last >> 32, self.marked) if self.marked is not None else None, "row": last & M32}
        wrong = {"content_wrong": bool(kind & W_CONTENT), "slot_wrong": bool(kind & W_SLOT)}
        if kind & W_CONTENT:
            wrong.update({"kv_head": info >> 12, "dim": (info >> 1) & 0x7FF, "part": "value" if info & 1 else "key"})
        detail = {"where": lay.name, "kind": "attention", "backend": lay.info["backend"], "finding": "kv_write_wrong",
                  "writes_checked": k[C_WN], "writes_with_wrong_content": k[C_WBAD],
                  "writes_to_another_slot": k[C_WSLOT], "latest": latest, "a_wrong_write": wrong,
                  "captured": {"row": latest["row"], "step": latest["step"]}, "read_window_steps": window,
                  "last_clean_read_steps": self.last_clean(lay.name),
                  "reading": "a sampled token's KV-cache slot does not hold the key and value the layer computed for "
                             "it, or they went to another slot than its position's block names: attention reads "
                             "wrong state for that position from now on"}
        return self.emit(lay, float("inf"), latest["row"], detail)


def check_call(binding, impl, query, key, value, kv_cache, md, output, output_scale=None) -> None:
    """After a backend call of a registered layer (binding: layer._sdcguard_attn)."""
    if binding is not None:
        binding.checks.check(binding, impl, query, key, value, kv_cache, md, output, output_scale)


__all__ = ["ATTN_Z", "SAMPLES", "COLS", "CAPM", "bound_consts", "sample_python", "buffers", "attn_check",
           "attn_check_triton", "run_case", "make_case", "recheck", "decode_state", "workspace_bytes", "AttnChecks",
           "why_not", "call_issue", "check_call"]
