"""The weight fingerprint and model digest against the reference's (tests/golden/weights.npz, from
serve_weights.fingerprint / model_digest on a model with 1, 2, 4 and 8-byte parameters), through the oracle; and
the recompute check's routing of torch.utils.checkpoint (install, partials held by modules, uninstall), which needs
no GPU."""
from __future__ import annotations

import functools
import hashlib
import json

import numpy as np
import torch

from oracle import fingerprint as F
from tests import _golden as G

W = G.load("weights.npz")
_DT = {"a.weight": (np.uint16, "bfloat16", (96, 64)), "a.bias": (np.uint16, "bfloat16", (96,)),
       "b.weight": (np.float16, "float16", (33, 96)), "c.scale": (np.float32, "float32", (7, 5)),
       "d.table": (np.float64, "float64", (4, 3)), "e.q": (np.int8, "int8", (40, 8))}


def params():
    out = []
    for n in (str(x) for x in W["names"]):
        npdt, name, shape = _DT[n]
        out.append((n, W["bits_" + n].view(npdt).reshape(shape), name))
    return out


def test_fingerprints_match_reference():
    for n, a, _ in params():
        assert F.fp2(F.fp2_words(a)).tolist() == W["fp_" + n].tolist(), n


def test_digest_text_matches_reference():
    h = hashlib.sha256()
    for n, a, dt in sorted(params(), key=lambda p: p[0]):
        f = F.fp2(F.fp2_words(a)).tolist()
        h.update(json.dumps([n, list(a.shape), dt, f]).encode())
    assert h.hexdigest()[:16] == str(W["digest"])


def test_recompute_routing_without_gpu():
    import torch.utils.checkpoint as tuc
    from sdcguard_amd import recompute as R
    orig_id = id(tuc.checkpoint)
    held = functools.partial(tuc.checkpoint, use_reentrant=False)
    m = torch.nn.Sequential(torch.nn.Linear(4, 4))
    m[0].ckpt = held
    rc = R.RecomputeCheck()
    rc.enabled = False                                  # the routing only: plain checkpoint underneath
    rc.install(m)
    assert tuc.checkpoint is R._dispatch and m[0].__dict__["ckpt"].func is R._dispatch
    x = torch.randn(3, 4, requires_grad=True)
    y = tuc.checkpoint(m, x, use_reentrant=False)
    y.sum().backward()
    assert x.grad is not None
    rc.uninstall()
    assert id(tuc.checkpoint) == orig_id and m[0].__dict__["ckpt"] is held
    assert R._dispatch(m, x, use_reentrant=False).shape == (3, 4)   # a reference kept after uninstall still works
    assert rc.stats["blocks_run"] == 0
