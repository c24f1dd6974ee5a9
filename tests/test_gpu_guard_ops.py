"""SDCGuard's dispatch route (SDCGuard(ops=True); the reference's __torch_dispatch__ -> _queue -> matmul_checks /
_grouped_checks, guard.py:1651-1805, :102-264) on a training step of a small model with a linear layer (addmm / mm),
an attention block (bmm) and MoE experts (torch._grouped_mm, tokens sorted by expert): a clean step raises nothing
and sees every kind of product in both passes; a fault added to one product's output -- a forward bmm, a forward
grouped product, a backward grouped product -- is reported at its op, batch or group, row and column block.

The fault is added by a dispatch mode entered before the guard's step: its handler runs the operator and changes
the result, so the guard's mode (on top of it) sees the changed result, as it would see a wrong GEMM's."""
from __future__ import annotations

import contextlib

import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode

pytestmark = pytest.mark.gpu

G, T, K, N, H = 4, 256, 256, 384, 4          # experts, tokens, width, expert outputs, heads
D = K // H
ENDS = (40, 120, 120, 256)                   # group ends: expert 2 gets no tokens


class _Fault(TorchDispatchMode):
    """Adds `delta` to the result of the `nth` call of aten op `name` (counting calls in this mode) at the position
    pick(result) returns; records the result's shape and the position."""

    def __init__(self, name: str, nth: int, pick, delta: float):
        super().__init__()
        self.name, self.nth, self.pick, self.delta = name, nth, pick, delta
        self.seen, self.hit = 0, None

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        out = func(*args, **(kwargs or {}))
        if func.overloadpacket.__name__ == self.name:
            self.seen += 1
            if self.seen == self.nth:
                at = self.pick(out)
                out[at] += self.delta
                self.hit = (tuple(out.shape), at)
        return out


class _Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.inp = torch.nn.Linear(K, K)
        self.experts = torch.nn.Parameter(torch.randn(G, N, K, generator=g) * K ** -0.5)
        self.offs = torch.tensor(ENDS, dtype=torch.int32)

    def forward(self, x):
        h = self.inp(x)                                             # addmm (backward: mm)
        q = h.view(T, H, D).transpose(0, 1).contiguous()            # (H, T, D)
        att = torch.softmax(torch.bmm(q, q.transpose(1, 2).contiguous()) * D ** -0.5, -1)
        h = torch.bmm(att, q).transpose(0, 1).reshape(T, K)
        w = self.experts.transpose(-2, -1)                          # (G, K, N), the layout MoE kernels take
        return torch._grouped_mm(h, w, offs=self.offs)


def _step(guard, model, x, fault=None):
    with (fault if fault is not None else contextlib.nullcontext()):
        with guard.at_step(1):
            model(x).float().square().mean().backward()
    return guard.flush()


def _setup():
    from sdcguard_amd.guard import SDCGuard
    torch.manual_seed(1)
    model = _Model().cuda().bfloat16()
    model.offs = model.offs.cuda()
    x = torch.randn(T, K, device="cuda").bfloat16()
    return SDCGuard(ops=True, every=0, fresh_signs=False), model, x


def _group_of(row: int) -> tuple:
    start = 0
    for g, end in enumerate(ENDS):
        if start <= row < end:
            return g, row - start
        start = max(start, end)
    raise AssertionError(row)


def test_clean_step_sees_every_product_and_raises_nothing():
    guard, model, x = _setup()
    res = _step(guard, model, x)
    print(guard.ops_seen, guard.stats, flush=True)
    assert guard.events == [] and res and all(r.ok for r in res)
    assert {"aten.addmm", "aten.mm", "aten.bmm", "aten._grouped_mm"} <= set(guard.ops_seen)
    # forward: 1 addmm, 2 bmm, 1 grouped; backward: mm for the linear layer, 4 bmm, 2 grouped (input, weights)
    assert guard.ops_seen["aten.bmm"] >= 6 and guard.ops_seen["aten._grouped_mm"] >= 3, guard.ops_seen


def test_fault_in_a_forward_bmm_is_located():
    guard, model, x = _setup()
    fault = _Fault("bmm", 2, lambda out: (2, 77, 45), 4.0)            # the second forward bmm: att @ q
    _step(guard, model, x, fault)
    print(fault.hit, [(e.layer, e.extra, e.row, e.col_block, e.z) for e in guard.events], flush=True)
    hit = [e for e in guard.events if e.layer == "aten.bmm"]
    assert len(hit) == 1 and hit[0].extra["pass"] == "forward" and hit[0].extra["batch"] == 2
    assert hit[0].row == 77 and hit[0].col_block == 0 and hit[0].z > 6


def test_fault_in_a_forward_grouped_product_is_located():
    guard, model, x = _setup()
    fault = _Fault("_grouped_mm", 1, lambda out: (130, 300), 3.0)     # token 130: expert 3 (rows 120 .. 255)
    _step(guard, model, x, fault)
    ev = [e for e in guard.events if e.layer == "aten._grouped_mm"]
    print(fault.hit, [(e.extra, e.row, e.col_block, e.z) for e in guard.events], flush=True)
    assert len(ev) == 1 and ev[0].extra["pass"] == "forward" and ev[0].extra["group"] == 3
    assert ev[0].row == 130 - 120 and ev[0].col_block == 300 // 128 and ev[0].z > 6


def test_fault_in_a_backward_grouped_product_is_located():
    guard, model, x = _setup()
    # the second grouped product runs in the backward pass: the input gradient (T, K) or the weight gradient
    # (G, K, N); either way the fault goes to row 5 and column 200 (of group 1 for the weight gradient)
    fault = _Fault("_grouped_mm", 2, lambda out: (5, 200) if out.dim() == 2 else (1, 5, 200), 2.0)
    _step(guard, model, x, fault)
    ev = [e for e in guard.events if e.layer == "aten._grouped_mm"]
    print(fault.hit, [(e.extra, e.row, e.col_block, e.z) for e in guard.events], flush=True)
    assert fault.hit is not None and len(ev) == 1 and ev[0].extra["pass"].startswith("backward") and ev[0].z > 6
    if len(fault.hit[0]) == 2:
        assert (ev[0].extra["group"], ev[0].row) == _group_of(5) and ev[0].col_block == 200 // 128
    else:
        assert ev[0].extra["group"] == 1 and ev[0].row == 5 and ev[0].col_block == 200 // 128
