"""The C-ABI library: it builds, loads without a GPU, and exports every symbol include/sdcguard_hip.h declares
(no compute calls here)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "sdcguard_hip.h")).read()
    return sorted(set(re.findall(r"^(?:int|int64_t|void)\s+(sdc_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = declared()
    assert "sdc_check_static" in names and "sdc_fingerprint3" in names


def test_library_exports_every_declared_symbol():
    from sdcguard_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing
    assert set(declared()) <= set(_lib.SIGNATURES), set(declared()) - set(_lib.SIGNATURES)


def test_workspace_sizes_are_host_only():
    from sdcguard_amd import _lib
    L = _lib.lib()
    assert L.sdc_check_static_workspace(0, 10, 10, 128) == 0
    ws = L.sdc_check_static_workspace(4096, 4096, 14336, 128)
    s = L.sdc_expected_splits(4096, 4096, 224)
    assert ws >= (s * 4096 * 224 + s * 2 * 4096) * 4


def test_product_refuses_cpu_tensors():
    """No CPU path: a check of CPU tensors raises instead of silently not running."""
    import torch
    from sdcguard_amd import _lib
    from sdcguard_amd.recompute import fingerprint
    with pytest.raises(_lib.HipLibraryError):
        fingerprint(torch.ones(10))


def _param_counts():
    """Number of parameters of every sdc_ function the header declares."""
    text = open(os.path.join(ROOT, "include", "sdcguard_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^(?:int|int64_t|void|const char\*)\s+(sdc_\w+)\s*\(([^)]*)\)\s*;", text, re.M):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def test_ctypes_signatures_take_as_many_arguments_as_the_header_declares():
    from sdcguard_amd import _lib
    counts = _param_counts()
    assert counts, "no declarations parsed"
    for name, n in counts.items():
        assert name in _lib.SIGNATURES, name
        assert len(_lib.SIGNATURES[name][1]) == n, (name, len(_lib.SIGNATURES[name][1]), n)
