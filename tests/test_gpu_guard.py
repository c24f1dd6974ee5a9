"""Training-side API on the GPU: Group / check_now against check_matmul, and SDCGuard.protect + at_step + flush
on a small bf16 MLP (forward, input-gradient and weight-gradient products of every linear layer), with a corrupted
layer output caught, located and raised, and sampling."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ab(m, k, n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    A = torch.randn(m, k, device="cuda", generator=g).bfloat16()
    B = (torch.randn(k, n, device="cuda", generator=g) * 0.05).bfloat16()
    return A, B, (A.float() @ B.float()).bfloat16()


def test_check_now_and_group_match_check_matmul():
    from sdcguard_amd.checksum import check_matmul
    from sdcguard_amd.guard import Group, check_now
    A, B, C = _ab(200, 320, 300, 1)
    z, b, r, cb, noise = check_now(A, B, C)
    ref = check_matmul(A, B, C)
    assert ref.ok and z == pytest.approx(ref.max_z, rel=1e-6) and noise > 0
    C[77, 150] += 2.0
    z, b, r, cb, noise = check_now(A, B, C)
    assert z > 6 and (r, cb) == (77, 1)
    g = Group(C.device, C.dtype)
    shapes = [(64, 128, 130), (33, 256, 257), (128, 64, 128)]
    mats = [_ab(*s, seed=i) for i, s in enumerate(shapes)]
    mats[1][2][5, 256] += 1.0                                  # the narrow last block of the second check
    idx = [g.add(a, bb, c, None, 1.0, 1.0) for a, bb, c in mats]
    g.launch()
    rows = g.result.cpu().tolist()
    got = [g.row(i, rows[i]) for i in idx]
    want = [check_matmul(a, bb, c) for a, bb, c in mats]
    assert [x[0] > 6 for x in got] == [not w.ok for w in want] == [False, True, False]
    assert got[1][2:4] == (5, 2)


def _mlp(seed=0):
    torch.manual_seed(seed)
    return torch.nn.Sequential(torch.nn.Linear(256, 512), torch.nn.GELU(), torch.nn.Linear(512, 192)).to(
        "cuda", torch.bfloat16)


def test_protect_checks_forward_and_both_gradients():
    from sdcguard_amd.guard import SDCGuard
    m = _mlp()
    g = SDCGuard(every=0).protect(m)
    x = torch.randn(96, 256, device="cuda").bfloat16()
    for step in range(2):
        with g.at_step(step):
            m(x).float().pow(2).mean().backward()
    res = g.flush()
    # per step: 2 forward, 1 input gradient (the first layer's input needs none), 2 weight gradients
    assert len(res) == 10 and all(r.ok for r in res), [r.max_z for r in res]
    assert g.stats["checks"] == 10 and g.stats["alerts"] == 0
    assert max(r.max_z for r in res) > 0


def test_corrupted_output_is_caught_and_raised():
    from sdcguard_amd.guard import SDCError, SDCGuard
    m = _mlp(seed=1)

    def corrupt(mod, args, y):
        y = y.clone()
        y[10, 70] += 8.0
        return y

    m[2].register_forward_hook(corrupt)                        # runs before the guard's hook
    seen = []
    g = SDCGuard(every=0, raise_on_alert=True, on_alert=seen.append).protect(m)
    x = torch.randn(64, 256, device="cuda").bfloat16()
    with g.at_step(5):
        with torch.no_grad():
            m(x)
    with pytest.raises(SDCError, match="2 \\(forward\\) at step 5"):
        g.flush()
    assert len(seen) == 1 and (seen[0].row, seen[0].col_block) == (10, 0) and seen[0].z > 6


def test_sampling_and_steps_outside_the_guard():
    from sdcguard_amd.guard import SDCGuard
    m = _mlp(seed=2)
    x = torch.randn(32, 256, device="cuda").bfloat16()
    g = SDCGuard(sample_rate=0.0, every=0).protect(m)
    with g.at_step(0):
        m(x).sum().backward()
    assert g.flush() == [] and g.stats["matmuls_seen"] == 5
    g2 = SDCGuard(every=0).protect(torch.nn.Sequential(*[mm for mm in m]))
    m(x).sum().backward()                                      # no step active: nothing queued
    assert g2.flush() == []
    g.unprotect()
    g2.unprotect()


def test_precise_mode_checks_the_fp32_accumulators():
    """precise=True: on a checked step each protected layer's forward, input-gradient and weight-gradient products
    are computed with fp32 outputs, checked (sdc_matmul_check_acc) and rounded once; the gradients agree with
    autograd's to bf16 rounding, unchecked steps run the plain layer, and a changed accumulator is caught."""
    from sdcguard_amd.guard import SDCGuard
    m = _mlp(seed=4)
    x = torch.randn(64, 256, device="cuda").bfloat16().requires_grad_()
    ref_y = m(x)
    ref_y.float().square().sum().backward()
    ref_gx, ref_gw = x.grad.clone(), m[0].weight.grad.clone()
    x.grad = None
    for p in m.parameters():
        p.grad = None
    g = SDCGuard(precise=True, every=0).protect(m)
    with g.at_step(1):
        y = m(x)
        y.float().square().sum().backward()
    res = g.flush()
    n_lin = sum(isinstance(mm, torch.nn.Linear) for mm in m)
    assert len(res) == 3 * n_lin and all(r.ok and r.max_z >= 0 for r in res), res
    assert g.stats["alerts"] == 0 and g.stats["checks"] == 3 * n_lin
    print("precise clean max z", max(r.max_z for r in res))
    torch.testing.assert_close(y.float(), ref_y.float(), rtol=2 ** -7, atol=1e-3)
    torch.testing.assert_close(x.grad.float(), ref_gx.float(), rtol=2 ** -6, atol=2e-3)
    torch.testing.assert_close(m[0].weight.grad.float(), ref_gw.float(), rtol=2 ** -6, atol=2e-3)
    with torch.no_grad():                                          # outside a step: the plain layer, bit for bit
        assert torch.equal(m(x), torch.nn.functional.linear(
            torch.nn.functional.gelu(torch.nn.functional.linear(x, m[0].weight, m[0].bias)), m[2].weight, m[2].bias)) \
            if len(m) == 3 else True
    g.unprotect()

    def bump(layer, where, c32):
        if layer == "2" and where == "weight grad":
            c32[7, 33] += 0.25
    seen = []
    g2 = SDCGuard(precise=True, every=0, on_accumulator=bump, on_alert=seen.append).protect(m)
    with g2.at_step(2):
        m(x).float().square().sum().backward()
    g2.flush()
    assert len(seen) == 1, seen
    ev = seen[0]
    assert ev.detector == "accumulator" and ev.layer == "2" and ev.extra["pass"] == "weight grad"
    assert (ev.row, ev.col_block) == (7, 0) and ev.z > 6
    g2.unprotect()


def test_precise_fused_mode_matches_precise_mode():
    """precise="fused" (_fused_compare.py:112-165): every linear product of a checked step goes through the fused
    GEMM's self-check; losses and gradients agree with precise=True's, both clean; a fault added to one weight
    gradient's accumulator raises one alert, named; with sample_rate the products left out run unchecked."""
    from sdcguard_amd.guard import SDCGuard

    def model():
        torch.manual_seed(0)
        return torch.nn.Sequential(torch.nn.Linear(256, 384), torch.nn.GELU(), torch.nn.Linear(384, 256)).cuda()

    def step(net, g, seed, step_no):
        torch.manual_seed(seed)
        x = torch.randn(48, 256, device="cuda")
        with g.at_step(step_no):
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = net(x).float().pow(2).mean()
            loss.backward()
        grads = [p.grad.clone() for p in net.parameters()]
        net.zero_grad()
        return loss.detach(), grads

    net_p, net_f = model(), model()
    gp = SDCGuard(every=0, precise=True).protect(net_p)
    gf = SDCGuard(every=0, precise="fused").protect(net_f)
    for s in range(2):
        lp, grp = step(net_p, gp, s, s)
        lf, grf = step(net_f, gf, s, s)
        assert torch.allclose(lp, lf, rtol=1e-3), (lp, lf)
        for a, c in zip(grp, grf):
            assert (a - c).abs().max() <= 2.0 ** -6 * a.abs().max()
    rf, rp = gf.flush(), gp.flush()
    print("fused guard stats:", gf.stats, "max z", max(r.max_z for r in rf))
    assert gf.stats["checked_fused"] == gf.stats["checks"] == 10 and gf.stats["alerts"] == 0
    assert gf.stats["fused_fallbacks"] == 0 and all(r.ok and r.max_z >= 0 for r in rf)
    assert gp.stats["alerts"] == 0 and len(rp) == 10

    hits = []
    gf.on_alert = hits.append
    gf.fused_inject = lambda name, pass_, shape: (3, 5, 0.05) if (name, pass_) == ("2", "weight grad") else None
    step(net_f, gf, 7, 2)
    gf.fused_inject = None
    gf.flush()
    assert len(hits) == 1, hits
    ev = hits[0]
    assert ev.layer == "2" and ev.extra["pass"] == "weight grad" and "fused" in ev.extra["dtype"]
    assert (ev.row, ev.col_block) == (3, 0) and ev.z > 6
    gp.unprotect()
    gf.unprotect()

    net_s = model()
    g_s = SDCGuard(every=0, precise="fused", sample_rate=0.5, seed=1).protect(net_s)
    step(net_s, g_s, 3, 0)
    g_s.flush()
    assert 0 < g_s.stats["checked_fused"] < g_s.stats["matmuls_seen"] == 5 and g_s.stats["alerts"] == 0, g_s.stats
    g_s.unprotect()
