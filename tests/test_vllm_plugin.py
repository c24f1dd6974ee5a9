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


# ---------------------------------------------------------------------------------------------------------------
# Attention through register(): stand-ins of vLLM's FlashAttention backend (a correct paged-attention forward in
# PyTorch, KV cache [blocks, kv heads, block size, 2 x head size]), its Attention layer and its model runner
# (load_model, execute_model running one decode step of every layer).

D_, HQ, HKV, NBLK, BS, REQ = 64, 4, 2, 64, 16, 4


def _fake_vllm_runner(fault: dict):
    import types as _t

    class FlashAttentionImpl:
        def __init__(self):
            self.num_heads, self.head_size, self.num_kv_heads, self.scale = HQ, D_, HKV, D_ ** -0.5
            self.sliding_window, self.kv_cache_dtype, self.attn_type = (-1, -1), "auto", "decoder"
            self.alibi_slopes, self.logits_soft_cap, self.sinks = None, 0, None

        def forward(self, layer, query, key, value, kv_cache, md, output=None, output_scale=None):
            T = md.num_actual_tokens
            slots = md.slot_mapping[:T]
            blk, off = slots // BS, slots % BS
            k_new = key[:T].clone()
            if fault.get("write"):                              # a wrong KV write: one bit of every new key
                k_new.view(torch.int16)[:, :, 3] ^= 1 << 9
            kv_cache[blk, :, off, :D_] = k_new
            kv_cache[blk, :, off, D_:] = value[:T]
            qsl, sls, bt = md.query_start_loc.tolist(), md.seq_lens.tolist(), md.block_table
            for r in range(len(sls)):
                i, L = qsl[r], sls[r]
                t = torch.arange(L, device=kv_cache.device)
                rows = kv_cache[bt[r, t // BS].long(), :, t % BS].float()       # [L, Hkv, 2D]
                if fault.get("read"):                           # the kernel read a changed value of the first key
                    rows = rows.clone()
                    rows[0, :, D_:] += 8.0
                for hq in range(HQ):
                    hk = hq // (HQ // HKV)
                    p = torch.softmax(rows[:, hk, :D_] @ query[i, hq].float() * self.scale, 0)
                    output[i, hq] = (p @ rows[:, hk, D_:]).to(output.dtype)
            return output

    class Attention(torch.nn.Module):
        def __init__(self, name):
            super().__init__()
            self.impl, self.layer_name = FlashAttentionImpl(), name

    class GPUModelRunner:
        def __init__(self):
            self.device = torch.device("cuda", 0)
            self.model_config = _t.SimpleNamespace(dtype=torch.bfloat16, max_model_len=4096)
            g = torch.Generator(device="cpu").manual_seed(3)
            self.gen = g
            self.caches = [(torch.randn(NBLK, HKV, BS, 2 * D_, generator=g) * 0.7).bfloat16().cuda()
                           for _ in range(2)]
            self.bt = torch.randperm(NBLK, generator=g)[:REQ * 8].view(REQ, 8).to(torch.int32).cuda()
            self.lens = [40, 57, 71, 90]

        def load_model(self):
            self.model = torch.nn.ModuleDict({"l0": Attention("model.layers.0.attn"),
                                              "l1": Attention("model.layers.1.attn")})

        def get_model(self):
            return self.model

        def execute_model(self, scheduler_output):
            self.lens = [n + 1 for n in self.lens]               # one new token per request
            T = REQ
            dev = self.device
            md = _t.SimpleNamespace(
                num_actual_tokens=T, causal=True,
                query_start_loc=torch.arange(T + 1, dtype=torch.int32, device=dev),
                seq_lens=torch.tensor(self.lens, dtype=torch.int32, device=dev), block_table=self.bt,
                slot_mapping=torch.tensor([int(self.bt[r, (L - 1) // BS]) * BS + (L - 1) % BS
                                           for r, L in enumerate(self.lens)], dtype=torch.int64, device=dev))
            for li, lay in enumerate(self.model.values()):
                q = (torch.randn(T, HQ, D_, generator=self.gen) * 0.5).bfloat16().to(dev)
                k = (torch.randn(T, HKV, D_, generator=self.gen) * 0.7).bfloat16().to(dev)
                v = (torch.randn(T, HKV, D_, generator=self.gen) * 0.7).bfloat16().to(dev)
                out = torch.empty(T, HQ, D_, dtype=torch.bfloat16, device=dev)
                lay.impl.forward(lay, q, k, v, self.caches[li], md, output=out)
            return None

    mods = {n: types.ModuleType(n) for n in ("vllm", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends",
                                             "vllm.v1.attention.backends.flash_attn", "vllm.v1.worker",
                                             "vllm.v1.worker.gpu_model_runner")}
    mods["vllm.v1.attention.backends.flash_attn"].FlashAttentionImpl = FlashAttentionImpl
    mods["vllm.v1.worker.gpu_model_runner"].GPUModelRunner = GPUModelRunner
    base, _ = _fake_vllm()
    for k in ("vllm.model_executor", "vllm.model_executor.layers", "vllm.model_executor.layers.linear"):
        mods[k] = base[k]
    return mods, GPUModelRunner


def _serve_steps(monkeypatch, fault: dict, steps: int = 6) -> list:
    from sdcguard_amd import vllm_plugin
    monkeypatch.setenv("SDCGUARD", "1")
    monkeypatch.setenv("SDCGUARD_POLL_EVERY", "1000")
    mods, Runner = _fake_vllm_runner(fault)
    for k, v in mods.items():
        monkeypatch.setitem(sys.modules, k, v)
    vllm_plugin.register()
    try:
        runner = Runner()
        runner.load_model()
        p = vllm_plugin.plugin_state()
        assert p.attn_report["checked"] == 2, p.attn_report
        for _ in range(steps):
            runner.execute_model(None)
        ev = vllm_plugin.poll(wait=True)
        g = p.guards[torch.device("cuda", 0)]
        print(p.errors, g._attn.stats, [(e.layer, e.extra.get("finding"), e.z) for e in ev], flush=True)
        assert not p.errors
        assert g._attn.stats["calls_checked"] == steps and g._attn.stats["samples"] > 0
        return ev
    finally:
        vllm_plugin.unregister()


@pytest.mark.gpu
def test_attention_checked_through_register_clean(monkeypatch):
    ev = _serve_steps(monkeypatch, {})
    assert ev == []


@pytest.mark.gpu
def test_attention_read_of_a_changed_value_is_flagged_through_register(monkeypatch):
    ev = _serve_steps(monkeypatch, {"read": True})
    found = {(e.layer, e.extra["finding"]) for e in ev}
    assert found == {("model.layers.0.attn", "output_wrong_or_misread"),
                     ("model.layers.1.attn", "output_wrong_or_misread")}, found
    assert all(e.z > 4 and e.extra["recheck"]["verdict"] in ("output_wrong", "not_rechecked") for e in ev)


@pytest.mark.gpu
def test_wrong_kv_write_is_flagged_through_register(monkeypatch):
    ev = _serve_steps(monkeypatch, {"write": True})
    found = {(e.layer, e.extra["finding"]) for e in ev}
    assert ("model.layers.0.attn", "kv_write_wrong") in found and ("model.layers.1.attn", "kv_write_wrong") in found
    w = next(e for e in ev if e.extra["finding"] == "kv_write_wrong")
    assert w.extra["a_wrong_write"]["content_wrong"] and w.extra["a_wrong_write"]["part"] == "key"


# ------------------------------------------------------------------------------------------------- MoE routers
MOE_E, MOE_K, MOE_T = 64, 6, 96


def _fake_moe_runner(fault: dict):
    """vLLM's router layout (FusedMoERouter.select_experts, subclassed by the routers) and a runner whose model has
    two MoE blocks with a router each: a DeepSeek-style grouped router and a softmax top-k one.  fault["route"]: the
    routers' kernel puts a wrong expert in every row's last slot."""
    import types as _t

    class FusedMoERouter:
        def select_experts(self, hidden_states, router_logits, topk_indices_dtype=None, *, input_ids=None):
            s = torch.softmax(router_logits.float(), -1) if self.scoring_func == "softmax" else \
                torch.sigmoid(router_logits.float())
            ch = s + self.e_score_correction_bias if self.e_score_correction_bias is not None else s
            groups = getattr(self, "num_expert_group", 0) or 0
            if groups:
                m = ch.shape[0]
                g = ch.view(m, groups, -1)
                gs = g.topk(2, -1).values.sum(-1) if self.e_score_correction_bias is not None else g.amax(-1)
                keep = torch.zeros(m, groups, dtype=torch.bool, device=ch.device)
                keep.scatter_(1, gs.topk(self.topk_group, -1).indices, True)
                ch = ch.masked_fill(~keep.repeat_interleave(MOE_E // groups, 1), float("-inf"))
            ids = ch.topk(self.top_k, -1).indices
            if fault.get("route"):
                ids[:, -1] = router_logits.float().argmin(-1)
            w = s.gather(1, ids)
            if self.renormalize:
                w = w / w.sum(-1, keepdim=True)
            scale = getattr(self, "routed_scaling_factor", 1.0) if type(self).__name__ != "FusedTopKRouter" else 1.0
            return (w * scale).float(), ids.to(torch.int32)

    class GroupedTopKRouter(FusedMoERouter):
        def __init__(self, bias):
            self.top_k, self.global_num_experts, self.scoring_func, self.renormalize = MOE_K, MOE_E, "sigmoid", True
            self.e_score_correction_bias, self.routed_scaling_factor = bias, 2.5
            self.num_expert_group, self.topk_group = 8, 3

    class FusedTopKRouter(FusedMoERouter):
        def __init__(self):
            self.top_k, self.global_num_experts, self.scoring_func, self.renormalize = MOE_K, MOE_E, "softmax", True
            self.e_score_correction_bias = None

    class MoEBlock(torch.nn.Module):
        def __init__(self, router):
            super().__init__()
            self.router = router

    class GPUModelRunner:
        def __init__(self):
            self.device = torch.device("cuda", 0)
            self.gen = torch.Generator(device="cpu").manual_seed(9)

        def load_model(self):
            bias = (torch.randn(MOE_E, generator=self.gen) * 0.03).cuda()
            self.model = torch.nn.ModuleDict({"moe0": MoEBlock(GroupedTopKRouter(bias)),
                                              "moe1": MoEBlock(FusedTopKRouter())})

        def get_model(self):
            return self.model

        def execute_model(self, scheduler_output):
            for blk in self.model.values():
                logits = (torch.randn(MOE_T + 8, MOE_E, generator=self.gen) * 2).bfloat16().cuda()   # 8 padding
                hidden = torch.zeros(MOE_T + 8, 16, device="cuda")
                blk.router.select_experts(hidden, logits)
            return None

    names = ("vllm", "vllm.v1", "vllm.v1.worker", "vllm.v1.worker.gpu_model_runner", "vllm.model_executor.layers",
             "vllm.model_executor.layers.fused_moe", "vllm.model_executor.layers.fused_moe.router",
             "vllm.model_executor.layers.fused_moe.router.fused_moe_router")
    mods = {n: types.ModuleType(n) for n in names}
    mods["vllm.v1.worker.gpu_model_runner"].GPUModelRunner = GPUModelRunner
    mods["vllm.model_executor.layers.fused_moe.router.fused_moe_router"].FusedMoERouter = FusedMoERouter
    base, _ = _fake_vllm()
    for k in ("vllm.model_executor", "vllm.model_executor.layers.linear"):
        mods[k] = base[k]
    mods["vllm.model_executor.layers"].linear = base["vllm.model_executor.layers.linear"]
    return mods, GPUModelRunner, FusedMoERouter, _t.SimpleNamespace(total_num_scheduled_tokens=MOE_T)


def _route_steps(monkeypatch, fault: dict, steps: int = 6) -> list:
    from sdcguard_amd import vllm_plugin
    monkeypatch.setenv("SDCGUARD", "1")
    monkeypatch.setenv("SDCGUARD_POLL_EVERY", "1000")
    mods, Runner, Router, sched = _fake_moe_runner(fault)
    for k, v in mods.items():
        monkeypatch.setitem(sys.modules, k, v)
    orig = Router.__dict__["select_experts"]
    vllm_plugin.register()
    try:
        assert Router.__dict__["select_experts"] is not orig
        runner = Runner()
        runner.load_model()
        p = vllm_plugin.plugin_state()
        assert p.route_report["checked"] == 2, p.route_report
        for _ in range(steps):
            runner.execute_model(sched)
        ev = vllm_plugin.poll(wait=True)
        rc = p.guards[torch.device("cuda", 0)]._route
        print(p.errors, rc.stats, [(e.layer, e.extra.get("finding"), e.extra.get("captured")) for e in ev], flush=True)
        assert not p.errors
        assert rc.stats["calls"] == steps and rc.stats["rows"] == 2 * steps
        return ev
    finally:
        vllm_plugin.unregister()
        assert Router.__dict__["select_experts"] is orig


@pytest.mark.gpu
def test_routing_checked_through_register_clean(monkeypatch):
    assert _route_steps(monkeypatch, {}) == []


@pytest.mark.gpu
def test_wrong_expert_from_a_router_is_flagged_through_register(monkeypatch):
    ev = _route_steps(monkeypatch, {"route": True})
    found = {(e.layer, e.extra["finding"]) for e in ev}
    assert found == {("moe0.router", "wrong_experts"), ("moe1.router", "wrong_experts")}, found
    assert all(e.extra["recheck"]["verdict"] == "output_wrong" and e.extra["captured"]["row"] < MOE_T for e in ev)
