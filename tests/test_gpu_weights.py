"""The scheduled weight scan (serve_weights.WeightScan through ServeGuard.weight_scan), the model digest and the
recompute check (recompute.RecomputeCheck) on the GPU: the digest against the reference's, a changed bit found
within one pass, moved and shared tensors left out rather than called changed, repair of a few changed values (and
not of many), asynchronous reads; the recompute check clean, on a block whose recompute differs, and through
SDCGuard(recompute=True)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.test_oracle_weights import W, params

pytestmark = pytest.mark.gpu


def test_model_digest_matches_reference():
    from sdcguard_amd.serve_weights import model_digest
    model = torch.nn.Module()
    for name, a, dt in params():
        mod_name, attr = name.split(".")
        if not hasattr(model, mod_name):
            model.add_module(mod_name, torch.nn.Module())
        t = torch.from_numpy(a.copy()).view(getattr(torch, dt)) if dt != "bfloat16" else \
            torch.from_numpy(a.copy().view(np.int16)).view(torch.bfloat16)
        getattr(model, mod_name).register_parameter(attr, torch.nn.Parameter(t.cuda(), requires_grad=False))
    d = model_digest(model)
    assert d == str(W["digest"]), (d, str(W["digest"]))
    with torch.no_grad():
        model.a.weight.view(torch.int16)[5, 7] ^= 1
    assert model_digest(model) != d


def _mlp(n=4, width=256, seed=0):
    torch.manual_seed(seed)
    layers = []
    for i in range(n):
        layers += [torch.nn.Linear(width, width), torch.nn.GELU()]
    return torch.nn.Sequential(*layers).cuda().bfloat16()


def test_scan_finds_a_flipped_bit_and_refresh_clears_it():
    from sdcguard_amd.serve import ServeGuard
    seen = []
    m = _mlp()
    g = ServeGuard(on_alert=seen.append).attach(m)
    scan = g.weight_scan(budget_mb=0.1)                  # about one layer per read
    assert scan.stats["entries"] == 4
    for _ in range(5):
        assert g.poll(wait=True) == []
    assert scan.stats["passes"] >= 1 and not scan.coverage()["never_compared"]
    with torch.no_grad():
        m[4].weight.view(torch.int16)[17, 33] ^= 1 << 3  # one mantissa bit of one weight
    found = []
    for _ in range(5):
        found += [e for e in g.poll(wait=True) if e.detector == "serve_weights"]
    assert len(found) == 1 and found[0].layer == "4" and found[0].extra["finding"] == "weights_changed", found
    assert scan.coverage()["changed"] == ["4"] and seen and seen[-1] is found[0]
    assert scan.refresh() == 4
    for _ in range(5):
        assert g.poll(wait=True) == []
    # asynchronous reads: a change shows at a later poll without waiting
    with torch.no_grad():
        m[2].bias.view(torch.int16)[3] ^= 1
    late = []
    for _ in range(12):
        late += g.poll(wait=False)
        torch.cuda.synchronize()
    assert [e.layer for e in late] == ["2"], late
    g.detach()


def test_moved_and_shared_tensors_are_left_out():
    from sdcguard_amd.serve_weights import WeightScan
    m = _mlp(n=3)
    scan = WeightScan(None, budget_mb=64)
    for i in (0, 2, 4):
        scan.add(f"l{i}", (lambda mod=m[i]: (mod.weight, mod.bias)), "checked", m[i])
    with torch.no_grad():                                # before the first comparison: the reference is retaken
        m[0].weight = torch.nn.Parameter(m[0].weight.detach().clone())
    assert scan.poll(wait=True) == [] and scan.stats["references_retaken"] == 1
    assert scan.poll(wait=True) == []
    with torch.no_grad():                                # after it: the layer is left out, never called changed
        m[2].weight = torch.nn.Parameter(m[2].weight.detach().clone())
    assert scan.poll(wait=True) == [] and "moved" in scan.not_scanned["l2"]
    alias = m[4].weight.detach().view(-1).view(m[4].weight.shape)    # another tensor object, the same memory
    scan.add("alias", (lambda: (alias,)), "other")
    assert scan.poll(wait=True) == []
    assert "shares its memory" in scan.not_scanned["alias"] and "shares its memory" in scan.not_scanned["l4"]


def test_repair_restores_a_few_values_not_many():
    from sdcguard_amd.serve_weights import WeightScan
    m = _mlp(n=2)
    scan = WeightScan(None, budget_mb=64, repair=True, host_allowance=1 << 30)
    for i in (0, 2):
        scan.add(f"l{i}", (lambda mod=m[i]: (mod.weight, mod.bias)), "checked", m[i])
    clean = m[0].weight.detach().clone()
    assert scan.poll(wait=True) == []
    with torch.no_grad():
        m[0].weight.view(torch.int16)[1, :3] ^= 0x4000
    ev = scan.poll(wait=True)                            # (the repair's record goes to events and on_alert)
    assert [e.extra["finding"] for e in ev] == ["weights_changed"], ev
    assert scan.events[-1].extra["finding"] == "weights_restored" and scan.events[-1].extra["values_changed"] == 3
    assert torch.equal(m[0].weight, clean) and scan.stats["repaired"] == 1
    assert scan.poll(wait=True) == []
    with torch.no_grad():
        m[2].weight.view(torch.int16)[:, :1] ^= 1        # 256 values: an update, not a fault
    ev = scan.poll(wait=True)
    assert [e.extra["finding"] for e in ev] == ["weights_changed"], ev
    assert scan.events[-1].extra["finding"] == "weights_restore_failed"
    assert scan.stats["repair_failed"] == 1 and scan.coverage()["changed"] == ["l2"]


class _Block(torch.nn.Module):
    def __init__(self, width=128, flaky=False):
        super().__init__()
        self.lin = torch.nn.Linear(width, width)
        self.flaky, self.runs = flaky, 0

    def forward(self, x):
        self.runs += 1
        y = torch.nn.functional.gelu(self.lin(x))
        if self.flaky and self.runs % 2 == 0:            # the recompute differs in one value
            y = y.clone()
            y[0, 0] += 1e-3
        return y


class _Net(torch.nn.Module):
    def __init__(self, flaky_at=None):
        super().__init__()
        self.blocks = torch.nn.ModuleList([_Block(flaky=i == flaky_at) for i in range(3)])
        self.head = torch.nn.Linear(128, 8)

    def forward(self, x):
        import torch.utils.checkpoint as tuc
        for b in self.blocks:
            x = tuc.checkpoint(b, x, use_reentrant=False)
        return self.head(x)


def test_recompute_check_clean_flaky_and_in_the_guard():
    from sdcguard_amd.guard import SDCGuard
    from sdcguard_amd.recompute import RecomputeCheck
    torch.manual_seed(0)
    net = _Net().cuda()
    x = torch.randn(16, 128, device="cuda")

    def step():
        net(x).square().sum().backward()

    rc = RecomputeCheck()
    cal = rc.calibrate(step, steps=2)
    assert cal["deterministic"] and cal["recomputes_compared"] == 6, cal
    cov = rc.coverage(net, step)
    assert cov["blocks_compared"] == 3 and 0.9 < cov["parameter_share_inside_compared_blocks"] < 1.0, cov
    flaky = _Net(flaky_at=1).cuda()
    hits = []
    rc2 = RecomputeCheck(on_alert=hits.append).install(flaky)
    flaky(x).square().sum().backward()
    ev = rc2.flush()
    rc2.uninstall()
    assert len(ev) == 1 and hits == ev and ev[0].extra["outputs_that_differ"] == [0], ev
    assert ev[0].extra["block_call"] == 2 and rc2.stats["mismatches"] == 1
    g = SDCGuard(recompute=True, every=0).protect(flaky)
    with g.at_step(3):
        flaky(x).square().sum().backward()
    g.flush()
    g.unprotect()
    rec = [e for e in g.events if e.detector == "recompute"]
    assert len(rec) == 1 and rec[0].step == 3, g.events
