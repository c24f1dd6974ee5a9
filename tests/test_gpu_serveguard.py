"""ServeGuard end to end on the GPU: attach -> forward -> poll -> detach on a small bf16 model, an injected fault
reported at its layer, row and block, polls that never stall, the check op under torch.compile, HIP-graph capture
and replay of a guarded forward, and a guarded forward that makes no host synchronisation (the reference's
tests/test_serve_no_sync.py)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _model(seed=0, bias=True):
    torch.manual_seed(seed)
    m = torch.nn.Sequential(torch.nn.Linear(256, 384, bias=bias), torch.nn.GELU(),
                            torch.nn.Linear(384, 200, bias=bias))
    return m.to("cuda", torch.bfloat16).eval()


def _x(rows=48, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(rows, 256, device="cuda", generator=g).bfloat16()


def test_attach_forward_poll_detach_clean():
    from sdcguard_amd.serve import ServeGuard
    m = _model()
    g = ServeGuard().attach(m)
    assert [lay["name"] for lay in g.layers] == ["0", "2"] and g.stats["layers"] == 2
    with torch.no_grad():
        for i in range(3):
            m(_x(seed=i))
    assert g.poll(wait=True) == []
    assert g.stats["checks_executed"] == 6 and g.checks_seen == {"0": 3, "2": 3}
    assert 0 < max(g.worst_seen.values()) < 6
    g.detach()
    assert not hasattr(m[0], "_sdcguard_slot") and len(m[0]._forward_hooks) == 0
    with torch.no_grad():
        m(_x())                                           # no guard left: nothing to count, nothing fails


def test_fault_in_a_layer_output_is_reported_where_it_is():
    from sdcguard_amd.serve import ServeGuard
    m = _model(seed=3)

    def corrupt(mod, args, out):                          # runs before the guard's hook (registered first)
        out = out.clone()
        out[17, 150] += 4.0
        return out

    m[2].register_forward_hook(corrupt)
    g = ServeGuard().attach(m)
    with torch.no_grad():
        m(_x(seed=5))
    ev = g.poll(wait=True)
    assert len(ev) == 1 and ev[0].layer == "2" and ev[0].row == 17 and ev[0].col_block == 1 and ev[0].z > 6
    assert g.stats["alerts"] == 1 and g.worst_seen["0"] < 6
    g.detach()


def test_polls_without_wait_report_the_previous_snapshot():
    from sdcguard_amd.serve import ServeGuard
    m = _model(seed=4)
    m[0].register_forward_hook(lambda mod, a, out: out.index_fill(1, torch.tensor([3], device="cuda"), 100.0))
    seen = []
    g = ServeGuard(on_alert=seen.append).attach(m)
    with torch.no_grad():
        m(_x(seed=6))
    assert g.poll() == []                                 # starts the copy, never waits
    torch.cuda.synchronize()
    ev = g.poll()                                         # the first snapshot has landed
    assert [e.layer for e in ev] == ["0"] and seen == ev
    with torch.no_grad():
        m(_x(seed=7))
    torch.cuda.synchronize()
    assert [e.layer for e in g.poll(wait=True)] == ["0"]  # the state was cleared by the earlier snapshot
    g.detach()


def test_share_and_unsupported_layers():
    from sdcguard_amd.serve import ServeGuard, select_layer
    m = torch.nn.Sequential(*[torch.nn.Linear(64, 64) for _ in range(8)]).to("cuda", torch.bfloat16)
    m.append(torch.nn.Linear(64, 64).cuda())              # fp32 weights: not checked
    g = ServeGuard().attach(m, share=0.5)
    picked = [i for i in range(8) if select_layer(i, 0.5)]
    assert [int(lay["name"]) for lay in g.layers] == picked
    assert "8" in g.unsupported
    g2 = ServeGuard().attach(m)                           # a second guard takes only the layers left over
    assert g2.unsupported[str(picked[0])].startswith("already")
    assert sorted(int(lay["name"]) for lay in g2.layers) == [i for i in range(8) if i not in picked]
    g2.detach()
    g.detach()


def test_check_op_under_torch_compile():
    from sdcguard_amd.serve import ServeGuard
    m = _model(seed=8)
    g = ServeGuard().attach(m)
    cm = torch.compile(m, backend="aot_eager", fullgraph=False)
    with torch.no_grad():
        for i in range(2):
            cm(_x(seed=10 + i))
    assert g.poll(wait=True) == [] and g.stats["checks_executed"] == 4
    g.detach()


def test_graph_replays_match_eager():
    """A guarded forward captured in a HIP graph: each replay (with eager work and a synchronisation between) adds
    the same checks and the same worst score as an eager forward of the same input."""
    from sdcguard_amd.serve import ServeGuard, decode_state
    m = _model(seed=9)
    x = _x(seed=11)
    g = ServeGuard().attach(m)
    with torch.no_grad():
        m(x)                                              # warm-up: constants, tables, workspaces
        torch.cuda.synchronize()
        eager = [decode_state(g.state("cuda")[s:s + 1])[0] for s in range(2)]
        g.state("cuda").zero_()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            m(x)                                          # warm-up on the capture stream (its workspace)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g.state("cuda").zero_()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            m(x)
        torch.cuda.synchronize()
        g.state("cuda").zero_()
        for r in range(1, 4):
            graph.replay()
            _ = (x.float() * 2).sum()                     # eager work between replays
            torch.cuda.synchronize()
            st = g.state("cuda")
            for slot in range(2):
                z, flat, _ = decode_state(st[slot:slot + 1])[0]
                assert (z, flat) == eager[slot][:2], (r, slot)
                assert int(st[slot, 2]) == r
    g.detach()


def test_guarded_forward_makes_no_host_sync():
    from sdcguard_amd.serve import ServeGuard
    m = _model(seed=12)
    g = ServeGuard().attach(m)
    x = _x(seed=13)
    with torch.no_grad():
        m(x)
        g.poll()
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            for _ in range(3):
                m(x)
                g.poll()
        finally:
            torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    g.detach()
