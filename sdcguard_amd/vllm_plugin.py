"""vLLM plugin entry point (reference: vllm_plugin.py:2239-2526, `register`; attention: :1675-1783).

register() is what vLLM's general-plugin loader calls in every process.  With SDCGUARD=1 it wraps:

  UnquantizedLinearMethod
    process_weights_after_loading(layer) after vLLM's own, the layer gets its serving-check constants (a slot in
                                         a per-device ServeGuard, LayerChecksums built on the GPU), if the layer
                                         is a bf16 / fp16 weight on a GPU and is among the SDCGUARD_SHARE of
                                         layers (golden-ratio spread, SDCGUARD_OFFSET); a reload reuses its slot
    apply(layer, x, bias)                vLLM's product, then the check of y against x: the sdcguard::check_static
                                         op while torch.compile traces (one opaque node, captured in HIP graphs),
                                         the library call in eager mode; no host synchronisation
  FlashAttentionImpl / TritonAttentionImpl
    forward(layer, q, k, v, kv_cache, metadata, output, ...)
                                         the backend's attention, then the sampled recompute of a registered layer
                                         (serve_attn.AttnChecks: one layer a step, from the paged KV cache) and the
                                         check of the step's own KV writes
  FusedMoERouter
    select_experts(hidden, logits, ...)  the router's experts and weights, then the check of a registered router's
                                         result against its policy recomputed from its logits (serve_route: one
                                         router a step, 2 rows)
  GPUModelRunner
    load_model()                         after vLLM's own, the model's attention layers and MoE routers are
                                         registered (before any graph is captured)
    execute_model(...)                   each model step is marked on the device before its work is queued and
                                         closed after it; results are read every SDCGUARD_POLL_EVERY steps (16)
                                         without waiting, and after SDCGUARD_POLL_SECONDS (2) with a wait

poll() returns the alerts found since the last poll.  SDCGUARD_Z sets the linear checks' alert line (default 6),
SDCGUARD_ATTN_Z the attention check's (default 4).  With SDCGUARD_REQUIRE set, anything that would leave the server
unchecked (SDCGUARD not 1, no vLLM layout this code knows) raises instead of serving.
"""
from __future__ import annotations

import importlib
import logging
import os
import time
from typing import Optional

import torch

log = logging.getLogger("sdcguard")


class RequirementNotMet(RuntimeError):
    """SDCGUARD_REQUIRE is set and the server would run unchecked."""


# the attention backends whose forward is followed by the check, and the model runners whose steps are marked
ATTN_BACKENDS = (("vllm.v1.attention.backends.flash_attn", "FlashAttentionImpl"),
                 ("vllm.v1.attention.backends.triton_attn", "TritonAttentionImpl"))
RUNNERS = ("vllm.v1.worker.gpu_model_runner", "vllm.v1.worker.gpu.model_runner")
ROUTER = ("vllm.model_executor.layers.fused_moe.router.fused_moe_router", "FusedMoERouter")


class _Plugin:
    """What register() installs: the wrapped methods, one ServeGuard per device, the layers' selection order and
    the step count."""

    def __init__(self, z: float, share: float, offset: int, attn_z: float = 4.0, poll_every: int = 16,
                 poll_seconds: float = 2.0):
        self.z, self.share, self.offset, self.attn_z = z, share, offset, attn_z
        self.poll_every, self.poll_seconds = max(1, int(poll_every)), float(poll_seconds)
        self.guards: dict = {}
        self.loaded = 0                  # eligible layers seen, in load order (a reload keeps a layer's number)
        self.steps = 0                   # model steps run
        self.last_poll = time.monotonic()
        self.attn_registered = False
        self.attn_report: dict = {}
        self.routers_registered = False
        self.route_report: dict = {}
        self.errors: dict = {}           # what failed in a hook -> times (the server keeps running)
        self.wrapped: list = []          # (class, attribute, original) to put back

    def guard(self, device):
        from .serve import ServeGuard
        g = self.guards.get(device)
        if g is None:
            g = self.guards[device] = ServeGuard(z=self.z)
        return g

    def after_loading(self, layer) -> None:
        from .checksum import UNIT_ROUNDOFF
        from .serve import select_layer
        w = getattr(layer, "weight", None)
        b = getattr(layer, "bias", None)
        b = b if isinstance(b, torch.Tensor) else None
        if not isinstance(w, torch.Tensor) or w.dim() != 2 or w.dtype not in UNIT_ROUNDOFF or not w.is_cuda:
            layer._sdcguard_why = "not a bf16 / fp16 weight on a GPU"
            return
        slot = getattr(layer, "_sdcguard_slot", 0)
        if slot:                                   # weights reloaded: new constants in the same slot
            g = self.guard(w.device)
            self._arm(layer, g, g.replace_layer(slot - 1, w, b))
            return
        number = getattr(layer, "_sdcguard_number", None)
        if number is None:
            number = layer._sdcguard_number = self.loaded
            self.loaded += 1
        if not select_layer(number, self.share, self.offset):
            layer._sdcguard_why = "not among the checked share of layers"
            return
        g = self.guard(w.device)
        name = getattr(layer, "prefix", "") or type(layer).__name__
        self._arm(layer, g, g.add_layer(layer, name, weight=w, bias=b))

    @staticmethod
    def _arm(layer, g, slot: int) -> None:
        # the guard and slot, not the op's arguments: a later layer can make the guard enlarge its device's state
        # and capture tensors, and the arguments are read from the guard on every call so that no layer keeps
        # writing into tensors the guard no longer polls
        layer._sdcguard_ref = (g, slot)
        layer.__dict__.pop("_sdcguard_why", None)

    @staticmethod
    def after_apply(layer, x, y, bias) -> None:
        from .serve import _op, check_static_impl
        ref = getattr(layer, "_sdcguard_ref", None)
        if ref is None or not isinstance(y, torch.Tensor):
            return
        g, slot = ref
        run = _op() if torch.compiler.is_compiling() else check_static_impl
        run(x.reshape(-1, x.shape[-1]), y.reshape(-1, y.shape[-1]), *g.op_args(slot, with_bias=bias is not None))

    def poll(self, wait: bool = False) -> list:
        events = []
        for g in self.guards.values():
            events += g.poll(wait=wait)
        return events

    def _failed(self, what: str, e: Exception) -> None:
        self.errors[what] = self.errors.get(what, 0) + 1
        log.warning("sdcguard: %s failed (%s: %s)", what, type(e).__name__, e)

    # -------------------------------------------------------------------------------------------- attention
    def after_attention(self, impl, layer, query, key, value, kv_cache, md, output, output_scale) -> None:
        from .serve_attn import check_call
        b = getattr(layer, "_sdcguard_attn", None)
        if b is None or md is None or output is None:
            return
        try:
            check_call(b, impl, query, key, value, kv_cache, md, output, output_scale)
        except Exception as e:  # noqa: BLE001  (never break serving: the layer goes unchecked from now on)
            layer.__dict__.pop("_sdcguard_attn", None)
            self._failed("an attention check", e)

    def register_attention(self, runner) -> dict:
        """After the model is loaded and before graphs are captured: its attention layers (modules with an `impl`
        and a `layer_name`) go to the device's guard, which numbers their turns and allocates their buffers."""
        if self.attn_registered:
            return self.attn_report
        self.attn_registered = True
        get = getattr(runner, "get_model", None)
        model = get() if callable(get) else getattr(runner, "model", None)
        found = [(n, m) for n, m in (model.named_modules() if model is not None else [])
                 if hasattr(m, "impl") and hasattr(m, "layer_name")]
        if not found:
            self.attn_report = {"checked": 0, "not_checked": {}, "why": "no attention layers found"}
            return self.attn_report
        mc = getattr(runner, "model_config", None)
        dtype = getattr(mc, "dtype", None)
        dev = getattr(runner, "device", None)
        if not isinstance(dev, torch.device):
            dev = next((p.device for p in model.parameters()), torch.device("cuda", torch.cuda.current_device()))
        ac = self.guard(dev).attn_checks(self.attn_z)
        for name, m in found:
            ac.add(m, m.impl, str(getattr(m, "layer_name", "") or name), dev, dtype)
        kv_dtype = dtype if dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
        ac.finalize(max_len=int(getattr(mc, "max_model_len", 0) or 32768), kv_dtype=kv_dtype)
        self.attn_report = {"checked": len(ac.layers), "not_checked": dict(ac.unsupported)}
        log.info("sdcguard: checking %d of %d attention layers (one a step)", len(ac.layers), len(found))
        return self.attn_report

    # ------------------------------------------------------------------------------------------------ routers
    def after_route(self, router, logits, weights, ids) -> None:
        from .serve_route import check_call
        b = getattr(router, "_sdcguard_route", None)
        if b is None:
            return
        try:
            check_call(b, logits, weights, ids)
        except Exception as e:  # noqa: BLE001  (never break serving: the router goes unchecked from now on)
            router.__dict__.pop("_sdcguard_route", None)
            self._failed("a routing check", e)

    def register_routers(self, runner) -> dict:
        """After the model is loaded and before graphs are captured: its MoE routers (the `router` of a module,
        with select_experts) go to the device's guard, which numbers their turns."""
        if self.routers_registered:
            return self.route_report
        self.routers_registered = True
        get = getattr(runner, "get_model", None)
        model = get() if callable(get) else getattr(runner, "model", None)
        found = []
        for name, m in (model.named_modules() if model is not None else []):
            r = getattr(m, "router", None)
            if r is not None and callable(getattr(r, "select_experts", None)) and \
                    getattr(r, "_sdcguard_route", None) is None:
                found.append((f"{name or type(m).__name__}.router", r))
        if not found:
            self.route_report = {"checked": 0, "not_checked": {}, "why": "no MoE routers found"}
            return self.route_report
        dev = getattr(runner, "device", None)
        if not isinstance(dev, torch.device):
            dev = next((p.device for p in model.parameters()), torch.device("cuda", torch.cuda.current_device()))
        rc = self.guard(dev).route_checks()
        for name, r in found:
            rc.add(r, name, dev)
        rc.finalize()
        self.route_report = {"checked": len(rc.layers), "not_checked": dict(rc.unsupported)}
        log.info("sdcguard: checking the routing of %d of %d MoE routers (one a step)", len(rc.layers), len(found))
        return self.route_report

    # ------------------------------------------------------------------------------------------------ steps
    def before_step(self, rows: Optional[int]) -> None:
        for g in self.guards.values():
            g.mark_step(self.steps + 1, rows)

    def after_step(self) -> None:
        for g in self.guards.values():
            g.end_step()
        self.steps += 1
        now = time.monotonic()
        late = now - self.last_poll >= self.poll_seconds
        if late or self.steps % self.poll_every == 0:
            self.last_poll = now
            self.poll(wait=late)


_PLUGIN: list = [None]


def _require(why: str) -> None:
    if os.environ.get("SDCGUARD_REQUIRE"):
        raise RequirementNotMet(f"sdcguard: {why}; SDCGUARD_REQUIRE is set, so the server does not start unchecked")
    log.warning("sdcguard: %s", why)


def _float_env(name: str, default: float) -> float:
    v = os.environ.get(name)
    try:
        return default if v is None else float(v)
    except ValueError:
        _require(f"{name}={v!r} is not a number")
        return default


def _rows_of_step(args, kwargs) -> Optional[int]:
    """The step's real tokens, from the scheduler output vLLM passes to execute_model (None: unknown)."""
    so = kwargs.get("scheduler_output", args[0] if args else None)
    n = getattr(so, "total_num_scheduled_tokens", None)
    return int(n) if isinstance(n, int) and n > 0 else None


def _wrap_attention(plugin: "_Plugin") -> list:
    """Follow each attention backend's forward with the check (vLLM calls it inside an opaque op of its own, eagerly
    and while graphs are captured).  Returns the classes wrapped."""
    done = []
    for module, cname in ATTN_BACKENDS:
        try:
            cls = getattr(importlib.import_module(module), cname)
            orig = cls.__dict__["forward"]
        except Exception as e:  # noqa: BLE001  (a vLLM build without this backend: nothing of it to check)
            log.info("sdcguard: vLLM's %s not found (%s); its attention is not checked", cname, e)
            continue

        def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, _orig=orig, **kwargs):
            out = _orig(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs)
            output = kwargs.get("output", args[0] if args else None)
            scale = kwargs.get("output_scale", args[1] if len(args) > 1 else None)
            plugin.after_attention(self, layer, query, key, value, kv_cache, attn_metadata,
                                   output if output is not None else out, scale)
            return out

        cls.forward = forward
        plugin.wrapped.append((cls, "forward", orig))
        done.append(cname)
    return done


def _wrap_router(plugin: "_Plugin") -> list:
    """Follow vLLM's MoE routers' select_experts with the routing check.  Returns the class wrapped."""
    module, cname = ROUTER
    try:
        cls = getattr(importlib.import_module(module), cname)
        orig = cls.__dict__["select_experts"]
    except Exception as e:  # noqa: BLE001  (a vLLM build without this router: no routing to check)
        log.info("sdcguard: vLLM's %s not found (%s); MoE routing is not checked", cname, e)
        return []

    def select_experts(self, hidden_states, router_logits, *args, _orig=orig, **kwargs):
        out = _orig(self, hidden_states, router_logits, *args, **kwargs)
        if isinstance(out, tuple) and len(out) == 2:
            plugin.after_route(self, router_logits, out[0], out[1])
        return out

    cls.select_experts = select_experts
    plugin.wrapped.append((cls, "select_experts", orig))
    return [cname]


def _wrap_runner(plugin: "_Plugin") -> list:
    """Register the attention layers and MoE routers after load_model; mark, close and read each model step around
    execute_model."""
    done = []
    for module in RUNNERS:
        try:
            GM = importlib.import_module(module).GPUModelRunner
        except Exception:  # noqa: BLE001
            continue
        orig_load, orig_exec = GM.__dict__.get("load_model"), GM.__dict__.get("execute_model")
        if orig_load is not None:
            def load_model(self, *args, _orig=orig_load, **kwargs):
                out = _orig(self, *args, **kwargs)
                try:
                    plugin.register_attention(self)
                except Exception as e:  # noqa: BLE001  (never break loading: attention goes unchecked)
                    plugin._failed("registering the attention layers", e)
                try:
                    plugin.register_routers(self)
                except Exception as e:  # noqa: BLE001  (never break loading: routing goes unchecked)
                    plugin._failed("registering the MoE routers", e)
                return out
            GM.load_model = load_model
            plugin.wrapped.append((GM, "load_model", orig_load))
        if orig_exec is not None:
            def execute_model(self, *args, _orig=orig_exec, **kwargs):
                if kwargs.get("dummy_run"):
                    return _orig(self, *args, **kwargs)
                try:
                    plugin.before_step(_rows_of_step(args, kwargs))
                except Exception as e:  # noqa: BLE001
                    plugin._failed("marking a step", e)
                try:
                    return _orig(self, *args, **kwargs)
                finally:
                    try:
                        plugin.after_step()
                    except Exception as e:  # noqa: BLE001  (never break serving)
                        plugin._failed("reading the checks", e)
            GM.execute_model = execute_model
            plugin.wrapped.append((GM, "execute_model", orig_exec))
        done.append(module)
    return done


def register() -> None:
    """vLLM general-plugin entry point; safe to call more than once."""
    if os.environ.get("SDCGUARD", "0") != "1":
        if os.environ.get("SDCGUARD_REQUIRE"):
            raise RequirementNotMet("sdcguard: SDCGUARD_REQUIRE is set but SDCGUARD isn't 1: nothing would be checked")
        return
    if _PLUGIN[0] is not None:
        return
    try:
        from vllm.model_executor.layers import linear as vlinear
        M = vlinear.UnquantizedLinearMethod
        orig_load, orig_apply = M.process_weights_after_loading, M.apply
    except (ImportError, AttributeError) as e:
        _require(f"vLLM layout not recognised ({type(e).__name__}: {e}); not checking anything")
        return
    z = _float_env("SDCGUARD_Z", 6.0)
    share = min(1.0, max(0.0, _float_env("SDCGUARD_SHARE", 1.0)))
    plugin = _PLUGIN[0] = _Plugin(z, share, int(_float_env("SDCGUARD_OFFSET", 0)), _float_env("SDCGUARD_ATTN_Z", 4.0),
                                  int(_float_env("SDCGUARD_POLL_EVERY", 16)), _float_env("SDCGUARD_POLL_SECONDS", 2.0))

    def process_weights_after_loading(self, layer):
        orig_load(self, layer)
        try:
            plugin.after_loading(layer)
        except Exception as e:  # noqa: BLE001  (a layer that cannot be checked must not stop the model loading)
            layer._sdcguard_why = f"{type(e).__name__}: {e}"
            log.warning("sdcguard: not checking %s: %s", getattr(layer, "prefix", "a layer"), e)

    def apply(self, layer, x, bias=None):
        y = orig_apply(self, layer, x, bias)
        plugin.after_apply(layer, x, y, bias)
        return y

    M.process_weights_after_loading = process_weights_after_loading
    M.apply = apply
    M._sdcguard_originals = (orig_load, orig_apply)
    plugin.attn_backends = _wrap_attention(plugin)
    plugin.routers = _wrap_router(plugin)
    plugin.runners = _wrap_runner(plugin)


def poll(wait: bool = False) -> list:
    """Alerts of every device's checks since the last poll (never waits unless asked)."""
    return [] if _PLUGIN[0] is None else _PLUGIN[0].poll(wait)


def unregister() -> None:
    """Put vLLM's methods back (tests, or a process that stops checking)."""
    p, _PLUGIN[0] = _PLUGIN[0], None
    if p is None:
        return
    from vllm.model_executor.layers import linear as vlinear
    M = vlinear.UnquantizedLinearMethod
    orig = getattr(M, "_sdcguard_originals", None)
    if orig is not None:
        M.process_weights_after_loading, M.apply = orig
        del M._sdcguard_originals
    for cls, attr, fn in reversed(p.wrapped):
        setattr(cls, attr, fn)
    p.wrapped.clear()
    for g in p.guards.values():
        g.detach()


def plugin_state() -> Optional[_Plugin]:
    return _PLUGIN[0]
