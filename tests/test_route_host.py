"""The router check's host side without a GPU: which vLLM routers it models and with what policy (the reference's
rules, serve_route.py:552-585), what it refuses and why, and that the product has no CPU path."""
from __future__ import annotations

import pytest
import torch

from sdcguard_amd import serve_route as sr


def _router(kind: str, **attrs):
    r = type(kind, (), {})()
    for k, v in attrs.items():
        setattr(r, k, v)
    return r


def test_plain_top_k_router_policy():
    pol, why = sr.policy_of(_router("FusedTopKRouter", top_k=2, global_num_experts=8, renormalize=True,
                                    routed_scaling_factor=3.0))
    assert why is None
    assert pol == {"k": 2, "scoring": 0, "renormalize": True, "bias": None, "groups": 0, "topk_group": 0,
                   "scale": 1.0, "experts": 8}                      # the fused top-k router does not scale


def test_grouped_router_policy_with_bias():
    bias = torch.randn(256)
    pol, why = sr.policy_of(_router("GroupedTopKRouter", top_k=8, global_num_experts=256, scoring_func="sigmoid",
                                    renormalize=True, e_score_correction_bias=torch.nn.Parameter(bias),
                                    routed_scaling_factor=2.5, num_expert_group=8, topk_group=4))
    assert why is None and pol["groups"] == 8 and pol["topk_group"] == 4 and pol["scoring"] == 1
    assert pol["scale"] == 2.5 and torch.equal(pol["bias"], bias)


def test_grouped_router_without_a_grouping_routes_as_plain_top_k():
    pol, _ = sr.policy_of(_router("GroupedTopKRouter", top_k=2, global_num_experts=8, scoring_func="sigmoid",
                                  routed_scaling_factor=2.0, num_expert_group=3, topk_group=1))
    assert (pol["groups"], pol["scoring"], pol["scale"]) == (0, 0, 1.0)
    pol, _ = sr.policy_of(_router("GroupedTopKRouter", top_k=2, global_num_experts=8, scoring_func="sigmoid",
                                  routed_scaling_factor=2.0, num_expert_group=3, topk_group=1,
                                  e_score_correction_bias=torch.zeros(8)))
    assert (pol["groups"], pol["scoring"], pol["scale"]) == (0, 1, 2.0)   # a bias keeps its scoring and scale


@pytest.mark.parametrize("attrs,why", [
    (dict(kind="CustomRouter", top_k=2), "CustomRouter"),
    (dict(kind="FusedTopKRouter", top_k=2, scoring_func="softplus"), "scoring function"),
    (dict(kind="FusedTopKRouter", top_k=2, eplb_state=object()), "expert load balancing"),
    (dict(kind="FusedTopKRouter", top_k=2, num_fused_shared_experts=1), "fused shared experts"),
    (dict(kind="FusedTopKRouter", top_k=2, _hash_indices_table=torch.zeros(3)), "hash routing"),
    (dict(kind="FusedTopKRouter", top_k=33, global_num_experts=64), "top-33"),
    (dict(kind="FusedTopKRouter", top_k=2, global_num_experts=4096), "top-2 of 4096"),
    (dict(kind="GroupedTopKRouter", top_k=8, global_num_experts=256, num_expert_group=8, topk_group=0),
     "8 expert groups choosing 0"),
    (dict(kind="GroupedTopKRouter", top_k=8, global_num_experts=256, num_expert_group=64, topk_group=1),
     "64 expert groups choosing 1"),
    (dict(kind="GroupedTopKRouter", top_k=2, global_num_experts=256, num_expert_group=128, topk_group=4),
     "128 expert groups"),
])
def test_routers_not_modeled_are_refused_with_a_reason(attrs, why):
    attrs = dict(attrs)
    pol, reason = sr.policy_of(_router(attrs.pop("kind"), **attrs))
    assert pol is None and why in reason


def test_no_cpu_path():
    from sdcguard_amd import _lib
    st = torch.zeros(1, sr.COLS, dtype=torch.int64)
    with pytest.raises(_lib.HipLibraryError):
        sr.route_check(torch.zeros(4, 8), torch.zeros(4, 2), torch.zeros(4, 2, dtype=torch.int32), 2, 0, True, None,
                       0, 0, 1.0, torch.ones(1, dtype=torch.int64), torch.zeros(1, dtype=torch.int64), st, 0, 1, 0,
                       torch.zeros(1, 6, dtype=torch.int64), torch.zeros(1, 8), torch.zeros(1, 2, dtype=torch.int64),
                       torch.zeros(1, 2))


def test_route_checks_refuse_cpu_routers_and_add_after_finalize():
    rc = sr.RouteChecks()
    r = _router("FusedTopKRouter", top_k=2, global_num_experts=8)
    assert rc.add(r, "r", "cpu") is None and rc.unsupported["r"] == "not on a GPU"
    rc.finalize()
    with pytest.raises(RuntimeError):
        rc.add(r, "r2", "cpu")


def test_check_call_ignores_calls_it_cannot_judge():
    """A binding-less call, a call whose ids are not the router's top-k, or 3-D logits: nothing is queued."""
    sr.check_call(None, torch.zeros(4, 8), torch.zeros(4, 2), torch.zeros(4, 2))

    class _B:
        class checks:
            @staticmethod
            def call_args(b):
                return (2,)
    sr.check_call(_B(), torch.zeros(4, 8), torch.zeros(4, 3), torch.zeros(4, 3))
    sr.check_call(_B(), torch.zeros(2, 4, 8), torch.zeros(4, 2), torch.zeros(4, 2))
