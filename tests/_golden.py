"""Loader of the golden fixtures written by tests/golden/make_golden.py (inputs as raw 16-bit words)."""
from __future__ import annotations

import os

import numpy as np

from oracle.lowp import bf16_from_bits

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name: str):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def words(f, name: str) -> np.ndarray:
    """uint16 words of stored array `name`, edits applied."""
    if name in f.files:
        return f[name]
    base = words(f, str(f[name + "_base"]))
    out = base.reshape(-1).copy()
    idx, val = f[name + "_edit"]
    out[idx] = val.astype(np.uint16)
    return out.reshape(base.shape)


def as_f32(w: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_from_bits(w).reshape(w.shape)
    return w.astype(np.uint16).view(np.float16).astype(np.float32)


def names(f):
    return [str(n) for n in f["names"]]


def f32_words(w: np.ndarray) -> np.ndarray:
    """float32 values stored as pairs of 16-bit words (low word first)."""
    return np.ascontiguousarray(w.astype(np.uint16)).reshape(-1).view(np.uint32).view(np.float32)
