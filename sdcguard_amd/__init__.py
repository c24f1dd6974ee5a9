"""sdcguard_amd: the verification hot path of sdcguard, MI355X-native (gfx950 HIP kernels behind a C ABI).

Public entry points follow the reference's (sdcguard/__init__.py): check_matmul / check_linear / matmul_zscores /
resolve (checksum), SDCGuard / Group / check_now (guard), ServeGuard and the sdcguard::check_static op (serve), the
vLLM plugin's register (vllm_plugin), fingerprint (recompute) and the weight fingerprint (serve_weights).  Every check runs in libsdcguard_hip.so; there is no CPU path.
"""
from .checksum import ABS_FLOOR, CheckResult, UNIT_ROUNDOFF, l1_floor_coef  # noqa: F401

__version__ = "0.1.0"


def __getattr__(name):
    if name in ("ServeGuard", "LayerChecksums"):
        from . import serve
        return getattr(serve, name)
    if name in ("check_matmul", "check_linear", "check_linear_rows", "matmul_zscores", "resolve"):
        from . import checksum
        return getattr(checksum, name)
    if name in ("SDCGuard", "Group", "check_now", "SDCError"):
        from . import guard
        return getattr(guard, name)
    if name == "fingerprint":
        from .recompute import fingerprint
        return fingerprint
    raise AttributeError(name)
