"""ctypes binding of libsdcguard_hip.so (the C ABI declared in include/sdcguard_hip.h).

The library is built in-tree by sdcguard_amd/csrc/build.py.  There is no fallback: if it is missing or cannot
be loaded, every check raises (a check that silently did not run would read as a clean result).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsdcguard_hip.so")

SDC_OK, SDC_EINVAL, SDC_EUNSUPPORTED, SDC_EWORKSPACE, SDC_ELAUNCH = 0, -1, -2, -3, -4
_NAMES = {SDC_EINVAL: "invalid argument", SDC_EUNSUPPORTED: "unsupported case", SDC_EWORKSPACE: "workspace too small",
          SDC_ELAUNCH: "HIP launch error"}

DT_BF16, DT_FP16 = 0, 1

_lock = threading.Lock()
_lib = [None]

P, I64, I32, F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

# name -> (restype, argtypes), in include/sdcguard_hip.h order
SIGNATURES = {
    "sdc_check_static_workspace": (I64, [I64, I64, I64, I64]),
    "sdc_check_static": (I32, [I32, P, I64, I64, P, I64, I64, I64, I64, I64, I64, P, I64, I64, I32, P, P, P, P, P,
                               P, P, P, I32, I64, F32, F32, P, P, I64, I64, I64, I64, I64, P, I64, P, I32, P, P, P]),
    "sdc_matmul_check_workspace": (I64, [I64, I64, I64, I64, I64, I64]),
    "sdc_matmul_check": (I32, [I32, P, I64, I64, I64, I64, P, I64, I64, I64, I64, P, I64, I64, I64, I64, I64, I64, I64,
                               I64, P, I32, I64, I64, I64, F32, F32, F32, F32, P, P, P, I64, P, P]),
    "sdc_matmul_check_acc_workspace": (I64, [I64, I64, I64, I64, I64, I64, I64]),
    "sdc_matmul_check_acc": (I32, [I32, P, I64, I64, I64, I64, P, I64, I64, I64, I64, P, I64, I64, I64, I64, I64, I64,
                                   I64, I64, P, I32, I64, I64, I64, F32, F32, F32, F32, F32, P, P, P, I64, P, P]),
    "sdc_matmul_check_acc_stats": (I32, [I32, P, I64, I64, P, I64, I64, P, I64, I64, I64, I64, I64, P, I32, F32, F32,
                                         F32, P, P, P, I64, P, P]),
    "sdc_fused_mm_workspace": (I64, [P, I64, I64, P, I64, I64, I64, I64, I64, I32]),
    "sdc_fused_mm": (I32, [I32, P, I64, I64, P, I64, I64, I64, I64, I64, P, I32, P, P, I64, P, I64, I64, F32, I32, P,
                           I64, P]),
    "sdc_fused_mm_checked": (I32, [I32, P, I64, I64, P, I64, I64, I64, I64, I64, P, I32, P, P, I64, F32, F32, F32, P, P,
                                   P, I64, I64, F32, I32, P, I64, P]),
    "sdc_fp8_quant_check_workspace": (I64, [I64]),
    "sdc_fp8_quant_check": (I32, [I32, P, I64, I64, I64, I64, P, I64, I64, I64, P, I64, I64, I32, P, P, P, P, I64, P,
                                  P, I64, P]),
    "sdc_moe_check_workspace": (I64, [I64, I64, I64]),
    "sdc_moe_check": (I32, [I32, P, I64, P, I64, P, I32, P, P, I64, I64, P, I64, I64, P, I64, I64, I64, I64, I64, I64,
                            I32, I32, P, I64, I64, F32, F32, F32, F32, P, P, P, P, P, P, P, P, I64, P]),
    "sdc_route_check": (I32, [P, I64, I32, P, I64, I32, P, I64, I32, P, I64, I64, I64, I32, I32, I32, I32, F32, F32,
                              P, P, I64, I64, P, P, P, P, P, P]),
    "sdc_expected_splits": (I64, [I64, I64, I64]),
    "sdc_linear_check_workspace": (I64, [I64, I64, I64]),
    "sdc_linear_check": (I32, [I32, P, I64, P, I64, P, I64, P, I64, I64, I64, P, I64, P, P, P, P, P, P, F32, F32,
                               P, I64, P, P, I32, P]),
    "sdc_parts_fragments_bytes": (I64, [I64, I64]),
    "sdc_parts_fragments": (I32, [P, I64, I64, I64, P, P]),
    "sdc_digit_fragments_bytes": (I64, [I64, I64]),
    "sdc_digit_fragments": (I32, [P, I64, I64, I64, P, P]),
    "sdc_grouped_check_workspace": (I64, [I64, I64, I64, I64, I64]),
    "sdc_grouped_constants_bytes": (I64, [I64, I64, I64, I64]),
    "sdc_grouped_constants_workspace": (I64, [I64, I64, I64, I64]),
    "sdc_grouped_constants": (I32, [I32, P, I64, I64, I64, I64, I64, I64, I64, P, I64, P, P, I64, P, I64, P]),
    "sdc_grouped_check_consts_workspace": (I64, [I64, I64, I64, I64, I64]),
    "sdc_grouped_check_consts": (I32, [I32, P, I64, I64, P, I64, P, I64, I64, I64, I64, I64, I64, P, I32, F32, F32, P,
                                       P, P, I64, P, P]),
    "sdc_grouped_check": (I32, [I32, P, I64, I64, P, I64, I64, I64, I64, P, I64, I64, I64, I64, I64, I64, P, P, I64,
                                F32, F32, P, P, P, I64, P, P]),
    "sdc_layer_constants_workspace": (I64, [I64, I64, I64]),
    "sdc_layer_constants": (I32, [I32, P, I64, I64, I64, I64, P, I64, P, P, I64, P, P, P, P, I64, P]),
    "sdc_quant_check_workspace": (I64, [I32, I64, I64, I64, I64]),
    "sdc_quant_check": (I32, [I32, P, I64, P, I64, P, P, P, I64, I64, I32, I64, I64, I64, I64, P, P, P, F32, F32, F32,
                              P, P, I64, P, P]),
    "sdc_fingerprint3": (I32, [P, I64, I32, I64, P, P]),
    "sdc_fingerprint2": (I32, [P, I64, I32, P, P]),
    "sdc_kv_fingerprint": (I32, [P, I64, I64, I64, I32, P, I64, P, P]),
    "sdc_attn_splits": (I64, [I64, I64]),
    "sdc_attn_check_workspace": (I64, [I64, I64, I64]),
    "sdc_attn_check": (I32, [I32, P, I64, I64, P, I64, I64, I64, I64, I64, P, I64, I64, I64, I64, I64, I64, I64,
                             P, I64, I64, P, I64, I64, P, P, I64, P, I64, I64, P, I64, P, I64, P, I64, I64, F32,
                             I64, F32, P, P, P, I64, P, P, I64, I32, P, I64, I32, I32, P, P]),
    "sdc_attn_check_noalloc": (I32, [I32, P, I64, I64, P, I64, I64, I64, I64, I64, P, I64, I64, I64, I64, I64, I64,
                                     I64, P, I64, I64, P, I64, I64, P, P, I64, P, I64, I64, P, I64, P, I64, P, I64,
                                     I64, F32, I64, F32, P, P, P, I64, P, P, I64, I32, I32, I32, P, P]),
    "sdc_mfma_layout_selftest": (I32, [P, P, P, P]),
    "sdc_last_error": (ctypes.c_char_p, []),
    "sdc_profile_enable": (I32, [I32]),
    "sdc_profile_reset": (I32, []),
    "sdc_profile_read": (I32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]),
}


class HipLibraryError(RuntimeError):
    """The HIP library is missing, cannot be loaded, or a call into it failed."""


def lib() -> ctypes.CDLL:
    if _lib[0] is None:
        with _lock:
            if _lib[0] is None:
                if not os.path.exists(LIB_PATH):
                    raise HipLibraryError(f"{LIB_PATH} is not built: run `python -m sdcguard_amd.csrc.build` "
                                          "(the checks have no fallback)")
                try:
                    L = ctypes.CDLL(LIB_PATH)
                except OSError as e:
                    raise HipLibraryError(f"cannot load {LIB_PATH}: {e}") from e
                for name, (res, args) in SIGNATURES.items():
                    f = getattr(L, name)
                    f.restype, f.argtypes = res, args
                _lib[0] = L
    return _lib[0]


def check(rc: int, what: str) -> None:
    if rc != SDC_OK:
        extra = ""
        if rc == SDC_ELAUNCH:
            extra = f": {lib().sdc_last_error().decode(errors='replace')}"
        raise HipLibraryError(f"{what}: {_NAMES.get(rc, 'error')} (status {rc}){extra}")


def stream_of(t: torch.Tensor) -> int:
    """The raw hipStream_t of the current stream of t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise HipLibraryError("sdcguard_amd checks run on the GPU only (tensor on "
                                  f"{t.device}); there is no CPU implementation in the product")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DT_BF16
    if dt == torch.float16:
        return DT_FP16
    raise HipLibraryError(f"unsupported dtype {dt}")


def profile_read(name: str):
    """(total ms, launches) of one kernel since the last sdc_profile_reset (waits for its events)."""
    ms, n = ctypes.c_double(0.0), ctypes.c_int64(0)
    check(lib().sdc_profile_read(name.encode(), ctypes.byref(ms), ctypes.byref(n)), "sdc_profile_read")
    return ms.value, n.value


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


_WS: dict = {}
_WS_LOCK = threading.Lock()


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A device workspace of at least `nbytes`, kept per (device, current stream) and grown when a call needs more,
    so steady-state calls allocate nothing (and a HIP-graph capture after a warm-up call reuses the same buffer).
    Calls on one stream are ordered, so they may share it; another stream gets its own."""
    dev = torch.device(device)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(dev).cuda_stream)
    with _WS_LOCK:
        buf = _WS.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)
            _WS[key] = buf
        return buf
