"""The FP8 quantization check on the GPU (sdc_fp8_quant_check through serve_fp8) against the reference's state rows
(tests/golden/fp8.npz), the oracle on full-size inputs, and the reference's serving flow (Fp8Checks: add,
mark_step, the calls, end_step, poll, alerts), in a captured graph too.  The state rows are integers and float
bits: compared exactly."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import serve_fp8 as of8
from tests.test_oracle_fp8 import NAMES, fp8_case

pytestmark = pytest.mark.gpu


def _x_dev(c):
    if c["dtc"] == 4:
        return torch.from_numpy(c["x"]).cuda()
    dt = torch.bfloat16 if c["dtc"] == 0 else torch.float16
    return torch.from_numpy(c["xw"].astype(np.uint16).view(np.int16)).view(dt).reshape(c["x"].shape).cuda()


def _run(c, x, xq, state=None):
    from sdcguard_amd import serve_fp8 as sf
    st = torch.zeros(1, sf.COLS, dtype=torch.int64, device="cuda") if state is None else state
    rows = torch.tensor([c["real"]], dtype=torch.int64, device="cuda")
    xs = torch.from_numpy(c["xs"]).cuda().reshape(-1, 1) if c["recipe"] == 2 else torch.from_numpy(c["xs"]).cuda()
    ub = None if c["ub"] is None else torch.from_numpy(c["ub"]).cuda()
    sref = None if c["sref"] is None else torch.from_numpy(c["sref"]).cuda()
    for s in c["steps"]:
        sf.quant_check(x, xq, xs, c["recipe"], ub, sref, rows, torch.tensor([s], dtype=torch.int64, device="cuda"),
                       st, 0, c["mult"])
    return st


@pytest.mark.parametrize("i", range(len(NAMES)))
def test_state_rows_match_reference(i):
    c = fp8_case(i)
    print(c["name"], flush=True)
    xq = torch.from_numpy(c["xq"]).cuda().view(torch.float8_e4m3fn)
    got = _run(c, _x_dev(c), xq)[0].cpu().tolist()
    assert got == c["state"].tolist(), (c["name"], got, c["state"].tolist())


@pytest.mark.parametrize("recipe", [1, 2])
def test_full_size_inputs_against_oracle(recipe):
    """A 4096 x 4096 bf16 input with 512 padding rows, over 40 steps: the scale from the real rows or from every
    row, and codes changed by 1 to 3 steps in random places; every state row as the oracle's."""
    from sdcguard_amd import serve_fp8 as sf
    g = torch.Generator(device="cuda").manual_seed(recipe)
    m, k, real = 4096, 4096, 3584
    x = (torch.randn(m, k, device="cuda", generator=g) * 2).bfloat16()
    x[real:] *= 8
    if recipe == 1:
        xs = (x[:real].float().abs().amax() / 448.0).reshape(1)
        xq = sf.quantize(x, xs, False)
    else:
        xs = (x.float().abs().amax(-1, keepdim=True) / 448.0).clamp(min=sf.MIN_SCALE)
        xq = sf.quantize(x, xs, True)
    rng = np.random.default_rng(recipe)
    state = torch.zeros(1, sf.COLS, dtype=torch.int64, device="cuda")
    want = np.zeros(8, np.int64)
    rows = torch.tensor([real], dtype=torch.int64, device="cuda")
    xh, xsh = x.float().cpu().numpy(), xs.float().cpu().numpy()
    for step in range(40):
        q = xq.clone()
        if step % 3 == 1:                            # corrupt one code of a sampled row
            r = int(sf.sample_rows(torch.tensor(step), torch.tensor(real))[step % 2])
            col = int(rng.integers(k))
            d = int(rng.integers(1, 4))
            code = int(q[r, col])
            q[r, col] = code + d if (code & 0x7F) < 0x7E - d else code - d
        use_xs = xs * 1.01 if step % 7 == 3 else xs
        sf.quant_check(x, q, use_xs, recipe, None, None, rows, torch.tensor([step], dtype=torch.int64,
                                                                            device="cuda"), state, 0)
        want = of8.quant_check(xh, q.cpu().numpy(), use_xs.cpu().numpy(), recipe, None, None, real, step, 1, want)
    got = state[0].cpu().tolist()
    print("state", got)
    assert got == want.tolist(), (got, want.tolist())
    assert got[of8.C_VALUES] > 0 and got[of8.C_SCALE] > 0


class _Quant:
    """A stand-in for a serving stack's FP8 input quantizer (the attributes recipe_of reads)."""

    def __init__(self, static=False, per_token=False, group=False):
        self.static, self.use_per_token_if_dynamic, self.is_group_quant = static, per_token, group
        self.group_shape = (-1, -1)


def test_fp8checks_flow_alerts_and_graph_capture():
    """Three layers (per tensor, per token, static) and one not checked (group scales): calls inside marked steps
    are judged, calls outside them are not; a scale taken over padding rows, a changed static scale and wrong codes
    become alerts naming the layer, the finding and the step's row; the same calls captured in a graph and replayed
    give the eager counters on every replay."""
    from sdcguard_amd import serve_fp8 as sf
    seen = []

    class _G:
        on_alert = staticmethod(seen.append)

    fc = sf.Fp8Checks(_G())
    dev = torch.device("cuda", 0)

    class _L:
        pass

    L = [_L() for _ in range(4)]
    s_static = torch.tensor([0.02], device=dev)
    a_t = fc.add(L[0], "tensor", _Quant(), None, dev)
    a_k = fc.add(L[1], "token", _Quant(per_token=True), None, dev)
    a_s = fc.add(L[2], "static", _Quant(static=True), s_static, dev)
    assert fc.add(L[3], "grouped", _Quant(group=True), None, dev) is None and "grouped" in fc.unsupported
    m, pad, k = 64, 16, 512
    x = (torch.randn(m + pad, k, device=dev) * 2).bfloat16()
    x[m:] *= 10
    real = m

    def calls(xt, s_pad):
        ok = (xt[:real].float().abs().amax() / 448.0).reshape(1)
        sf.check_call(a_t, xt, sf.quantize(xt, s_pad if s_pad is not None else ok, False),
                      s_pad if s_pad is not None else ok)
        tok = (xt.float().abs().amax(-1, keepdim=True) / 448.0).clamp(min=sf.MIN_SCALE)
        sf.check_call(a_k, xt, sf.quantize(xt, tok, True), tok)
        sf.check_call(a_s, xt, sf.quantize(xt, s_static, False), s_static)

    calls(x, None)                                   # outside a step: not judged
    fc.mark_step(5, real)
    calls(x, None)
    fc.end_step()
    assert fc.poll(wait=True) == [] and fc.stats["calls"] == 3
    fc.mark_step(6, real)
    calls(x, (x.float().abs().amax() / 448.0).reshape(1))       # per-tensor scale over the padding rows
    s_static.mul_(1.5)                                           # a static scale changed since load
    calls(x, None)
    fc.end_step()
    ev = fc.poll(wait=True)
    found = {e.layer: e.extra["finding"] for e in ev}
    print(found, fc.stats)
    assert found == {"tensor": "scale_from_outside_rows", "static": "static_scale_changed"}, found
    assert next(e for e in ev if e.layer == "tensor").extra["captured"] == {"step": 6, "row": None, "every_row": True}
    assert len(seen) == 2 and fc.coverage()["layers_checked"] == 3
    s_static.div_(1.5)

    # the calls in a captured graph: replays judge like eager calls
    st = fc.tables[dev].state
    fc.mark_step(9, real)
    calls(x, None)
    torch.cuda.synchronize()
    st.zero_()
    calls(x, None)
    torch.cuda.synchronize()
    eager = st.clone()
    st.zero_()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        calls(x, None)                               # warm-up on the capture stream (workspace for this stream)
        torch.cuda.synchronize()
        st.zero_()
        with torch.cuda.graph(graph, stream=s):
            calls(x, None)
    torch.cuda.synchronize()
    st.zero_()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(st, eager), (rep, st[:3], eager[:3])
        _ = (x.float() * 2).sum().item()             # the program's own work between replays
        st.zero_()
    fc.end_step()
    fc.detach()
