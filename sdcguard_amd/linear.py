"""Both block checksums of one linear layer y = x @ W^T (+ b), from one read of y (sdc_linear_check).

The column-block check is the serving check (serve.py:301-396: every row of y against x . B2 per block of 128 output
columns, B2 the layer's block sums made once by LayerChecksums); the row-block check is the training check of the
transposed product (checksum.py:435-530 on W, x^T, y^T, b[:, None]: every column of y against W_j . (block sums of
x) per block of 128 rows).  One library call runs both and reads y once; the scores, keys and counts are those of
sdc_check_static and sdc_matmul_check.  bf16 layers only (fp16 layers take the two checks separately).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib
from .checksum import ABS_FLOOR, CheckResult, CheckStat, resolve, sign_table
from .serve import STATE_COLS, LayerChecksums, _kmajor_parts, _packed_consts, decode

BLOCK = 128


def check_linear_both(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], y: torch.Tensor,
                      cs: LayerChecksums, *, z: float = 6.0, abs_floor: float = ABS_FLOOR,
                      state: Optional[torch.Tensor] = None, row_result: Optional[torch.Tensor] = None,
                      concurrent: bool = False, col_scores: Optional[torch.Tensor] = None,
                      row_scores: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Queue both checks of y = linear(x, weight, bias) on the current stream (no host sync).  cs: the layer's
    LayerChecksums (block 128).  Returns (state, row_result): the column check's int64[4] state row (worst key, key
    with noise, checks, unjudged) and the row check's int64[3] result row (worst key, key with noise, unjudged);
    pass zeroed ones to fold several calls into one.  concurrent: run the column check's GEMM and the x pass's
    finishing step on a side stream beside the x pass and the row check's GEMM; the default (False) keeps every
    kernel on the current stream, where the row check's GEMM runs that finishing step in its spare workgroups (on
    MI355X for the 4096 x 4096 x 14336 layer the one-stream form is the faster: the column GEMM fills every CU, so
    the side stream only adds the cost of its fork and join)."""
    _lib.require_gpu(x, weight, y)
    if y.dtype != torch.bfloat16 or x.dtype != y.dtype or weight.dtype != y.dtype:
        raise _lib.HipLibraryError("check_linear_both takes bf16 layers (fp16: check_static_impl and "
                                   "check_linear_rows)")
    if cs.bs != BLOCK:
        raise ValueError(f"the layer's checksums use blocks of {cs.bs}, not {BLOCK}")
    x2, y2 = x.reshape(-1, x.shape[-1]), y.reshape(-1, y.shape[-1])
    m, k = x2.shape
    n = y2.shape[1]
    if weight.shape != (n, k):
        raise ValueError(f"weight {tuple(weight.shape)} does not map x ({m} x {k}) to y ({m} x {n})")
    for t in (x2, weight, y2):
        if t.stride(-1) != 1:
            raise ValueError("x, weight and y must have a contiguous last dimension")
    dev = y2.device
    if state is None:
        state = torch.zeros(STATE_COLS, dtype=torch.int64, device=dev)
    if row_result is None:
        row_result = torch.zeros(3, dtype=torch.int64, device=dev)
    t = cs.tensors(True)
    parts, scale, b2n, b2max, bmax, bmax_bias, bsum = t[0], t[3], t[4], t[5], t[6], t[7], t[8]
    P = _kmajor_parts(parts, scale, cs.nb, y2.dtype)
    packed = _packed_consts(scale, b2n, b2max, bmax, bmax_bias, bsum)
    wn = getattr(cs, "wnorm", None)
    if wn is None or wn.shape != (2, n):
        raise ValueError("the layer's checksums carry no row norms of W (LayerChecksums makes them)")
    L = _lib.lib()
    frag = _fragments(P, 2 * cs.nb, k)
    nbytes = int(L.sdc_linear_check_workspace(m, k, n))
    ws = _lib.workspace(dev, nbytes)
    rc = L.sdc_linear_check(
        _lib.DT_BF16, x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0), y2.data_ptr(), y2.stride(0),
        _lib.ptr(bias), m, k, n, P.data_ptr(), P.stride(1), _lib.ptr(frag), packed.data_ptr(), wn.data_ptr(),
        sign_table(dev).data_ptr(), state.data_ptr(), row_result.data_ptr(), float(z), float(abs_floor),
        ws.data_ptr(), ws.numel(), _lib.ptr(col_scores), _lib.ptr(row_scores), 1 if concurrent else 0,
        _lib.stream_of(y2))
    if rc == _lib.SDC_EUNSUPPORTED:
        # a layout the one-pass kernels do not read (rows not 16-byte aligned): the two checks, one after the other
        _separately(x2, weight, bias, y2, cs, z, abs_floor, state, row_result, col_scores, row_scores)
        return state, row_result
    _lib.check(rc, "sdc_linear_check")
    return state, row_result


def _fragments(P: torch.Tensor, ncols: int, k: int) -> Optional[torch.Tensor]:
    """The layer's parts in the register-streamed GEMM's fragment order (sdc_parts_fragments), made once and kept on
    the parts tensor (so they live as long as the constants they copy); None where that GEMM does not apply (depth
    not a multiple of 256, part columns not 16-byte aligned)."""
    if k % 256 or P.stride(1) % 8 or P.data_ptr() % 16:
        return None
    key = (P.data_ptr(), P._version, ncols, k)
    hit = getattr(P, "_sdc_frag", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    L = _lib.lib()
    out = torch.empty(int(L.sdc_parts_fragments_bytes(ncols, k)) // 2, dtype=torch.int16, device=P.device)
    _lib.check(L.sdc_parts_fragments(P.data_ptr(), P.stride(1), ncols, k, out.data_ptr(), _lib.stream_of(P)),
               "sdc_parts_fragments")
    try:
        P._sdc_frag = (key, out)
    except (AttributeError, RuntimeError):
        pass
    return out


def _separately(x2, weight, bias, y2, cs, z, abs_floor, state, row_result, col_scores, row_scores) -> None:
    from .checksum import linear_rows_operands, matmul_zscores
    from .serve import check_static_impl
    check_static_impl(x2, y2, *cs.tensors(True), state.view(1, -1), 0, z, abs_floor, scores_out=col_scores)
    rs = None if row_scores is None else row_scores.view(1, *row_scores.shape)
    matmul_zscores(*linear_rows_operands(x2, weight, bias, y2), z=z, abs_floor=abs_floor, out=row_result,
                   scores_out=rs)


def resolve_both(state: torch.Tensor, row_result: torch.Tensor, m: int, n: int,
                 z: float = 6.0) -> Tuple[Optional[CheckResult], Optional[CheckResult]]:
    """Read both rows (one device-to-host copy each): the column check's worst checksum as a CheckResult (row,
    col_block = block of output columns) and the row check's (row = output column, col_block = block of rows)."""
    s = state.cpu().tolist()
    zc, flat, noise = decode(s[0], s[1])
    nb = -(-n // BLOCK)
    finite = math.isfinite(zc)
    col = CheckResult(ok=finite and zc <= z, max_z=zc, nonfinite=not finite, batch=None, row=(flat // 2) // nb,
                      col_block=(flat // 2) % nb, noise=noise)
    row = resolve([CheckStat(row_result, n, -(-m // BLOCK), False, z)], z)[0]
    return col, row
