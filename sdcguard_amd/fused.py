"""The precise check fused into the matmul (reference: fused.py).

A linear layer's matmul computed by the library's own MFMA GEMM (fused_check.hip) whose epilogue, before rounding,
either reduces every 128-column block of each output row to four float64 numbers (plain sum, signed sum, sum of
squares, sum of absolute values: `fused_mm`, scored by `zscores_from_stats` against x . (block sums of W) in
float64), or scores the check itself (`fused_mm_checked`: the expected side x . (block sums of W) accumulated in the
same depth loop from three 16-bit parts of each block sum on MFMA, with a compensated fp32 sum, and precise mode's
noise model plus that side's own rounding).  The layer's output comes from the same fp32 accumulator, so the
matmul runs once and nothing reads the product back.

Trade-offs, as in the reference: on checked steps the layer's output comes from this GEMM, not hipBLASLt (the same
fp32 accumulation rounded the same way, in another summation order, so output bits can differ in the last place
from a hipBLASLt run); nn.Linear layers under protect() only.  The reference's Triton tiling knobs (bm, bk,
num_warps) are accepted and ignored: the tiling is fixed (256 x 256 tiles, depth 32 per stage).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import checksum as cs

BLOCK = 128                        # checksum block width (fused.py:41)
NX = 16                            # columns of the narrow dot: 2 blocks x 3 parts x 2 sums, padded (fused.py:260)
_SIGNS: dict = {}


def available(x: torch.Tensor) -> bool:
    """x is a bf16/fp16 tensor on a GPU (fused.py:45-50).  The HIP library itself is required: a call without it
    raises instead of falling back."""
    return isinstance(x, torch.Tensor) and x.dtype in (torch.bfloat16, torch.float16) and x.is_cuda


def _signs_for(n: int, device, epoch: int) -> torch.Tensor:
    """The signed-checksum pattern of every output column: the 128-wide pattern repeated over full blocks, then the
    remainder block's own pattern (fused.py:53-68)."""
    key = (n, str(device), epoch)
    s = _SIGNS.get(key)
    if s is None:
        nfull, rem = divmod(n, BLOCK)
        parts = []
        if nfull:
            parts.append(cs._signs(BLOCK, "cpu", epoch).double().repeat(nfull))
        if rem:
            parts.append(cs._signs(rem, "cpu", epoch).double())
        s = torch.cat(parts).to(device) if parts else torch.zeros(0, dtype=torch.float64, device=device)
        if len(_SIGNS) > 64:
            _SIGNS.clear()
        _SIGNS[key] = s
    return s


def _shapes(A: torch.Tensor, B: torch.Tensor, bias: Optional[torch.Tensor]):
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise ValueError(f"shape mismatch: A{tuple(A.shape)} B{tuple(B.shape)}")
    if bias is not None and tuple(bias.shape) != (B.shape[1],):
        raise ValueError(f"bias must have shape ({B.shape[1]},), not {tuple(bias.shape)}")


def _require(A: torch.Tensor) -> None:
    if not available(A):
        raise RuntimeError("the fused check needs a bf16/fp16 tensor on a GPU (and the HIP library)")


def _bias_arg(bias: Optional[torch.Tensor], dt: torch.dtype):
    """The bias as the kernel reads it: of A's dtype, or fp32 (any other dtype is converted to fp32, exactly for
    the 16-bit ones); contiguous."""
    if bias is None:
        return None, 0
    if bias.dtype not in (dt, torch.float32):
        bias = bias.float()
    return bias.contiguous(), int(bias.dtype == torch.float32)


def _inject(inject):
    if inject is None:
        return 0, 0, 0.0, 0
    r, c, v = inject
    return int(r), int(c), float(v), 1


def fused_mm(A: torch.Tensor, B: torch.Tensor, bias: Optional[torch.Tensor] = None, epoch: int = 0,
             inject: Optional[tuple] = None, bm: int = 64, bk: int = 32, num_warps: int = 8):
    """C = A @ B + bias in A's dtype, and (m, ceil(n/128), 4) float64 block statistics of the fp32 result before
    rounding: plain sum, signed sum, sum of squares, sum of absolute values (fused.py:116-170).  A: (m, k), B: (k, n),
    any strides; bias: (n,), added in fp32 before rounding.  inject=(row, col, value) adds value to one accumulator
    element before rounding (experiments)."""
    from . import _lib
    _shapes(A, B, bias)
    _require(A)
    M, K = A.shape
    N = B.shape[1]
    if B.dtype != A.dtype:
        B = B.to(A.dtype)
    C = torch.empty((M, N), dtype=A.dtype, device=A.device)
    nb = -(-N // BLOCK)
    stats = torch.empty((M, nb, 4), dtype=torch.float64, device=A.device)
    if M == 0 or N == 0:
        return C, stats
    _lib.require_gpu(A, B, bias)
    b, b32 = _bias_arg(bias, A.dtype)
    L = _lib.lib()
    ws_bytes = int(L.sdc_fused_mm_workspace(A.data_ptr(), A.stride(0), A.stride(1), B.data_ptr(), B.stride(0),
                                            B.stride(1), M, K, N, 0))
    ws = _lib.workspace(A.device, ws_bytes)
    im, inn, iv, on = _inject(inject)
    rc = L.sdc_fused_mm(_lib.dtype_code(A.dtype), A.data_ptr(), A.stride(0), A.stride(1), B.data_ptr(), B.stride(0),
                        B.stride(1), M, K, N, None if b is None else b.data_ptr(), b32,
                        cs.sign_table(A.device, epoch).data_ptr(), C.data_ptr(), C.stride(0), stats.data_ptr(),
                        im, inn, iv, on, ws.data_ptr(), ws_bytes, _lib.stream_of(A))
    _lib.check(rc, "sdc_fused_mm")
    return C, stats


def fused_linear(x2: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None, **kw):
    """y = x2 @ w.T + bias and its block statistics (fused.py:173-176)."""
    return fused_mm(x2, w.t(), bias, **kw)


def zscores_from_stats(A: torch.Tensor, B: torch.Tensor, stats: torch.Tensor, bias: Optional[torch.Tensor] = None,
                       *, z: float = 6.0, nfma: Optional[int] = None, epoch: int = 0,
                       abs_floor: float = cs.ABS_FLOOR, out: Optional[torch.Tensor] = None,
                       scores_out: Optional[torch.Tensor] = None) -> cs.CheckStat:
    """Precise mode's check of C = A @ B + bias with C's block statistics taken from fused_mm instead of a stored
    fp32 C (fused.py:181-235).  A: (m, k) bf16/fp16; B: (k, n), for example w.T.  Queued without waiting; resolve()
    reads it."""
    from . import _lib
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise ValueError(f"shape mismatch: A{tuple(A.shape)} B{tuple(B.shape)}")
    M, K = A.shape
    N = B.shape[1]
    nb = -(-N // BLOCK)
    if tuple(stats.shape) != (M, nb, 4) or stats.dtype != torch.float64:
        raise ValueError(f"stats must be ({M}, {nb}, 4) float64, not {tuple(stats.shape)} {stats.dtype}")
    if B.dtype != A.dtype:
        B = B.to(A.dtype)
    if out is None:
        out = torch.zeros(3, dtype=torch.int64, device=A.device)
    if M == 0 or N == 0:
        return cs.CheckStat(result=out, m=max(M, 1), nb=max(nb, 1), batched=False, z=float(z))
    _lib.require_gpu(A, B, stats, bias)
    if K == 0:                                             # one zero column, as the precise check pads
        A = A.new_zeros(M, 1)
        B = B.new_zeros(1, N)
        K = 1
    b, b32 = _bias_arg(bias, A.dtype)
    st = stats if stats.stride(2) == 1 else stats.contiguous()
    L = _lib.lib()
    ws_bytes = int(L.sdc_matmul_check_acc_workspace(1, 1, 1, M, K, N, BLOCK))
    ws = _lib.workspace(A.device, ws_bytes)
    rc = L.sdc_matmul_check_acc_stats(
        _lib.dtype_code(A.dtype), A.data_ptr(), A.stride(0), A.stride(1), B.data_ptr(), B.stride(0), B.stride(1),
        st.data_ptr(), st.stride(0), st.stride(1), M, K, N, None if b is None else b.data_ptr(), b32,
        float(nfma or 0), float(z), float(abs_floor), cs.sign_table(A.device, epoch).data_ptr(), out.data_ptr(),
        ws.data_ptr(), ws_bytes, None if scores_out is None else scores_out.data_ptr(), _lib.stream_of(A))
    _lib.check(rc, "sdc_matmul_check_acc_stats")
    return cs.CheckStat(result=out, m=M, nb=nb, batched=False, z=float(z))


def check_linear_fused(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None, *, z: float = 6.0,
                       nfma: Optional[int] = None, epoch: int = 0, inject: Optional[tuple] = None):
    """(y, CheckResult): the linear layer's output from the fused kernel and the precise check of its fp32
    accumulator (fused.py:238-246).  x may have leading batch dimensions."""
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    y, stats = fused_linear(x2, w, bias, epoch=epoch, inject=inject)
    st = zscores_from_stats(x2, w.to(x2.dtype).t(), stats, bias, z=z, nfma=nfma, epoch=epoch)
    return y.reshape(*lead, w.shape[0]), cs.resolve([st], z)[0]


def fused_mm_checked(A: torch.Tensor, B: torch.Tensor, bias: Optional[torch.Tensor] = None, *, z: float = 6.0,
                     nfma: Optional[int] = None, epoch: int = 0, abs_floor: float = cs.ABS_FLOOR,
                     inject: Optional[tuple] = None, bm: int = 64, bk: int = 32, num_warps: int = 8,
                     out: Optional[torch.Tensor] = None, scores_out: Optional[torch.Tensor] = None,
                     expected_out: Optional[torch.Tensor] = None):
    """C = A @ B + bias from the fused kernel, and the check of its fp32 accumulator scored in the kernel
    (fused.py:462-546): cs.CheckStat, decoded by checksum.resolve like every other check.  No float64 on the
    expected side, no host sync.  A: (m, k), B: (k, n), any strides; bias (n,) added in fp32 before rounding.
    scores_out ((m, nb, 2) fp32) and expected_out ((m, nb, 2) float64), optional, receive every block's scores and
    expected sides."""
    from . import _lib
    _shapes(A, B, bias)
    _require(A)
    M, K = A.shape
    N = B.shape[1]
    if B.dtype != A.dtype:
        B = B.to(A.dtype)
    nb = -(-N // BLOCK)
    if out is None:
        out = torch.zeros(3, dtype=torch.int64, device=A.device)
    if M == 0 or N == 0 or K == 0:                         # fused.py:489-494: nothing to judge
        C, _ = fused_mm(A, B, bias) if M and N else (torch.empty((M, N), dtype=A.dtype, device=A.device), None)
        return C, cs.CheckStat(result=out, m=max(M, 1), nb=max(nb, 1), batched=False, z=float(z))
    _lib.require_gpu(A, B, bias)
    C = torch.empty((M, N), dtype=A.dtype, device=A.device)
    b, b32 = _bias_arg(bias, A.dtype)
    L = _lib.lib()
    ws_bytes = int(L.sdc_fused_mm_workspace(A.data_ptr(), A.stride(0), A.stride(1), B.data_ptr(), B.stride(0),
                                            B.stride(1), M, K, N, 1))
    ws = _lib.workspace(A.device, ws_bytes)
    im, inn, iv, on = _inject(inject)
    rc = L.sdc_fused_mm_checked(
        _lib.dtype_code(A.dtype), A.data_ptr(), A.stride(0), A.stride(1), B.data_ptr(), B.stride(0), B.stride(1),
        M, K, N, None if b is None else b.data_ptr(), b32, cs.sign_table(A.device, epoch).data_ptr(), C.data_ptr(),
        C.stride(0), float(nfma or 0), float(z), float(abs_floor), out.data_ptr(),
        None if scores_out is None else scores_out.data_ptr(),
        None if expected_out is None else expected_out.data_ptr(), im, inn, iv, on, ws.data_ptr(), ws_bytes,
        _lib.stream_of(A))
    _lib.check(rc, "sdc_fused_mm_checked")
    return C, cs.CheckStat(result=out, m=M, nb=nb, batched=False, z=float(z))
