"""The attention check's entry point that allocates nothing (sdc_attn_check_noalloc, through the C ABI) against
the entry point with a workspace (sdc_attn_check): the same state rows, capture rows and per-dimension scores, on
two calls in a row, the second with a smaller input (fewer keys, fewer samples, another head size)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _both(c, samples, step):
    from sdcguard_amd import serve_attn as SA
    D = c["q"].shape[-1]
    out = []
    for noalloc in (False, True):
        b = SA.buffers(DEV, 1, D, 256, c["q"].dtype, samples=samples)
        zs = torch.full((samples, D), float("nan"), device=DEV)
        b["ctrl"][0], b["ctrl"][1] = step, 1
        args = (c["q"], c["o"], c["kv"], c["key"], c["val"], c["qsl"], c["seq_lens"], c["bt"], c["slots"],
                b["state"], 0, b["ctrl"], 1, 0, c["scale"], -1, SA.ATTN_Z, b["capm"], b["capq"], b["capo"],
                b["capkv"], b["capkvm"])
        if noalloc:
            SA.attn_check_noalloc(*args, True, True, samples=samples, scores_out=zs)
        else:
            SA.attn_check(*args, b["ws"], True, True, samples=samples, scores_out=zs)
        torch.cuda.synchronize()
        out.append((b["state"].cpu(), b["capm"].cpu(), b["capq"].cpu(), b["capo"].cpu(), zs.cpu(),
                    b["capkvm"].cpu()))
    return out


def _kept_problems(c, m, q, o, k) -> list:
    """What is wrong with a kept row: claimed, over the line, and holding its own (row, head)'s q and o."""
    from sdcguard_amd import serve_attn as SA
    from sdcguard_amd.stepchecks import f32_of
    meta = [int(v) for v in m[0].tolist()]
    if not meta[SA.CM_CLAIM]:
        return ["no row kept"]
    row, head, D = meta[SA.CM_ROW], meta[SA.CM_HEAD], c["q"].shape[-1]
    out = []
    if not f32_of(meta[SA.CM_Z]) > SA.ATTN_Z:
        out.append(("score", f32_of(meta[SA.CM_Z])))
    if not torch.equal(q[0, :D], c["q"][row, head].float().cpu()) or not torch.equal(o[0, :D],
                                                                                  c["o"][row, head].float().cpu()):
        out.append(("kept q / o", row, head))
    kept = bool(meta[SA.CM_KEPT])
    if (int(k[0]) == 1) != kept or (kept and int(k[2]) != meta[SA.CM_POS] - meta[SA.CM_LO] + 1):
        out.append(("kept keys", k.tolist(), meta))
    return out


def test_noalloc_matches_the_workspace_entry_point_on_two_calls_the_second_smaller():
    from sdcguard_amd import serve_attn as SA
    big = SA.make_case(DEV, torch.bfloat16, D=128, Hq=8, Hkv=2, NB=400, lens=((4000, 1), (2100, 3), (90, 1)),
                       seed=21, padded_rows=1)
    big["o"][:, 5, 70] += 0.6
    small = SA.make_case(DEV, torch.bfloat16, D=64, Hq=4, Hkv=2, NB=12, lens=((70, 1), (21, 6), (3, 3), (0, 0)),
                         seed=22)
    small["key"][:, 0, 3] += 1.0                     # wrong KV writes
    for c, samples, step in ((big, 16, 3), (small, 4, 1)):
        (s0, m0, q0, o0, z0, k0), (s1, m1, q1, o1, z1, k1) = _both(c, samples, step)
        assert torch.equal(s0, s1), (samples, s0, s1)
        assert torch.equal(torch.nan_to_num(z0, nan=-1.0), torch.nan_to_num(z1, nan=-1.0))
        # the kept row: the first sample over the line to claim it (samples race for it), so either call may keep
        # another of the samples over the line; each keeps a whole, correct one, and the same one gives the same
        if int(m0[0, SA.CM_CLAIM]) or int(m1[0, SA.CM_CLAIM]):
            assert not _kept_problems(c, m0, q0, o0, k0) and not _kept_problems(c, m1, q1, o1, k1), \
                (_kept_problems(c, m0, q0, o0, k0), _kept_problems(c, m1, q1, o1, k1))
            if torch.equal(m0[0, SA.CM_ROW:SA.CM_HEAD + 1], m1[0, SA.CM_ROW:SA.CM_HEAD + 1]):
                assert torch.equal(m0, m1) and torch.equal(k0, k1) and torch.equal(q0, q1) and torch.equal(o0, o1)
        assert int(s0[0, SA.C_CALLS]) == 1


def test_noalloc_rejects_nothing_within_the_limits_and_leaves_its_counters_at_zero():
    """Every accepted call fits the static workspace; repeated calls keep giving the workspace entry point's
    answer (the counters the last workgroup of each sample resets)."""
    from sdcguard_amd import _lib
    from sdcguard_amd import serve_attn as SA
    L = _lib.lib()
    for samples in (1, 4, 16, 64, 1024):
        for keys in (16, 4096, 1 << 20):
            assert L.sdc_attn_check_workspace(samples, keys, 256) <= SA.SCRATCH_BYTES
    c = SA.make_case(DEV, torch.float16, D=128, Hq=2, Hkv=1, NB=90, lens=((1300, 1), (40, 2)), seed=23)
    ref = None
    for _ in range(3):
        (s0, *_r0), (s1, *_r1) = _both(c, 8, 2)
        assert torch.equal(s0, s1)
        ref = s0 if ref is None else ref
        assert torch.equal(s1, ref)
