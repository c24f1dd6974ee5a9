"""The vLLM plugin's register() against a stand-in of the vLLM module layout it patches (vLLM itself is not
installed here): the environment switches on the CPU; on the GPU, weights loaded through the patched method get
their constants, the patched apply checks every product, a corrupted product is reported, a reload keeps the slot,
and unregister() puts vLLM's methods back."""
from __future__ import annotations

import sys
import types

import pytest
import torch


def _fake_vllm(corrupt=None):
    """Modules vllm.model_executor.layers.linear with an UnquantizedLinearMethod like vLLM's (its apply is the plain
    product; `corrupt`, if set, is applied to the product, as a faulty GEMM would)."""
    class UnquantizedLinearMethod:
        def process_weights_after_loading(self, layer):
            layer.loaded = getattr(layer, "loaded", 0) + 1

        def apply(self, layer, x, bias=None):
            y = torch.nn.functional.linear(x, layer.weight, bias)
            return corrupt(y) if corrupt is not None else y

    mods = {}
    for name in ("vllm", "vllm.model_executor", "vllm.model_executor.layers", "vllm.model_executor.layers.linear"):
        mods[name] = types.ModuleType(name)
    mods["vllm.model_executor.layers.linear"].UnquantizedLinearMethod = UnquantizedLinearMethod
    mods["vllm.model_executor.layers"].linear = mods["vllm.model_executor.layers.linear"]
    return mods, UnquantizedLinearMethod


@pytest.fixture
def fake_vllm(monkeypatch):
    holder = {}

    def install(corrupt=None):
        mods, M = _fake_vllm(corrupt)
        for k, v in mods.items():
            monkeypatch.setitem(sys.modules, k, v)
        holder["M"] = M
        return M
    yield install
    from sdcguard_amd import vllm_plugin
    if vllm_plugin.plugin_state() is not None:
        vllm_plugin.unregister()


def test_register_is_off_without_sdcguard(monkeypatch, fake_vllm):
    from sdcguard_amd import vllm_plugin
    M = fake_vllm()
    monkeypatch.delenv("SDCGUARD", raising=False)
    monkeypatch.delenv("SDCGUARD_REQUIRE", raising=False)
    orig = M.apply
    vllm_plugin.register()
    assert M.apply is orig and vllm_plugin.plugin_state() is None
    monkeypatch.setenv("SDCGUARD_REQUIRE", "1")
    with pytest.raises(vllm_plugin.RequirementNotMet):
        vllm_plugin.register()


def test_register_without_vllm_refuses_only_when_required(monkeypatch):
    from sdcguard_amd import vllm_plugin
    monkeypatch.setitem(sys.modules, "vllm", None)            # import vllm fails
    monkeypatch.setenv("SDCGUARD", "1")
    monkeypatch.delenv("SDCGUARD_REQUIRE", raising=False)
    vllm_plugin.register()
    assert vllm_plugin.plugin_state() is None
    monkeypatch.setenv("SDCGUARD_REQUIRE", "1")
    with pytest.raises(vllm_plugin.RequirementNotMet):
        vllm_plugin.register()


def _layer(n, k, seed, bias=True):
    torch.manual_seed(seed)
    lin = torch.nn.Linear(k, n, bias=bias).to("cuda", torch.bfloat16)
    lin.prefix = f"model.layers.{seed}.mlp"
    return lin


@pytest.mark.gpu
def test_patched_methods_check_every_product(monkeypatch, fake_vllm):
    from sdcguard_amd import vllm_plugin
    monkeypatch.setenv("SDCGUARD", "1")
    state = {"bad": False}

    def corrupt(y):
        if state["bad"]:
            y = y.clone()
            y[3, 140] += 4.0
        return y

    M = fake_vllm(corrupt)
    vllm_plugin.register()
    vllm_plugin.register()                                   # twice: no double wrapping
    meth = M()
    layers = [_layer(384, 256, 0), _layer(256, 384, 1, bias=False)]
    for lay in layers:
        meth.process_weights_after_loading(lay)
        assert lay.loaded == 1 and hasattr(lay, "_sdcguard_ref")
    x = torch.randn(48, 256, device="cuda").bfloat16()
    h = meth.apply(layers[0], x, layers[0].bias)
    meth.apply(layers[1], torch.nn.functional.gelu(h), None)
    assert vllm_plugin.poll(wait=True) == []
    g = vllm_plugin.plugin_state().guards[torch.device("cuda", 0)]
    assert g.stats["checks_executed"] == 2
    state["bad"] = True
    meth.apply(layers[0], x, layers[0].bias)
    ev = vllm_plugin.poll(wait=True)
    assert len(ev) == 1 and ev[0].layer == "model.layers.0.mlp" and (ev[0].row, ev[0].col_block) == (3, 1)
    # a reload keeps the slot and takes the new weights
    with torch.no_grad():
        layers[1].weight.mul_(0.5)
    meth.process_weights_after_loading(layers[1])
    state["bad"] = False
    meth.apply(layers[1], torch.nn.functional.gelu(h), None)
    assert vllm_plugin.poll(wait=True) == [] and len(g.layers) == 2
    vllm_plugin.unregister()
    assert not hasattr(M, "_sdcguard_originals")


@pytest.mark.gpu
def test_layers_armed_before_the_state_grows_still_report(monkeypatch, fake_vllm):
    """A layer deeper than the first allocation (k > 8192) makes the guard enlarge its device's state and capture
    tensors; a fault in a layer loaded before that is still reported, and both layers' checks are counted."""
    from sdcguard_amd import vllm_plugin
    monkeypatch.setenv("SDCGUARD", "1")
    state = {"bad": False}

    def corrupt(y):
        if state["bad"] and y.shape[1] == 384:
            y = y.clone()
            y[5, 300] += 8.0
        return y

    M = fake_vllm(corrupt)
    vllm_plugin.register()
    meth = M()
    first, deep = _layer(384, 256, 2), _layer(128, 9216, 3, bias=False)
    meth.process_weights_after_loading(first)
    g = vllm_plugin.plugin_state().guards[torch.device("cuda", 0)]
    rows_before = g._rows[torch.device("cuda", 0)]
    meth.process_weights_after_loading(deep)
    assert g._rows[torch.device("cuda", 0)] is not rows_before       # the deep layer enlarged the device's rows
    x = torch.randn(16, 256, device="cuda").bfloat16()
    state["bad"] = True
    meth.apply(first, x, first.bias)
    meth.apply(deep, torch.randn(16, 9216, device="cuda").bfloat16(), None)
    ev = vllm_plugin.poll(wait=True)
    assert len(ev) == 1 and ev[0].layer == "model.layers.2.mlp" and (ev[0].row, ev[0].col_block) == (5, 2)
    assert g.stats["checks_executed"] == 2
    vllm_plugin.unregister()
