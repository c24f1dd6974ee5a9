"""vLLM plugin entry point (reference: vllm_plugin.py:2239-2367, `register`).

register() is what vLLM's general-plugin loader calls in every process.  With SDCGUARD=1 it wraps two methods of
vLLM's UnquantizedLinearMethod:

  process_weights_after_loading(layer)   after vLLM's own, the layer gets its serving-check constants (a slot in
                                         a per-device ServeGuard, LayerChecksums built on the GPU), if the layer
                                         is a bf16 / fp16 weight on a GPU and is among the SDCGUARD_SHARE of
                                         layers (golden-ratio spread, SDCGUARD_OFFSET); a reload reuses its slot
  apply(layer, x, bias)                  vLLM's product, then the check of y against x: the sdcguard::check_static
                                         op while torch.compile traces (one opaque node, captured in HIP graphs),
                                         the library call in eager mode; no host synchronisation

poll() returns the alerts found since the last poll.  SDCGUARD_Z sets the alert line (default 6).  With
SDCGUARD_REQUIRE set, anything that would leave the server unchecked (SDCGUARD not 1, no vLLM layout this code
knows) raises instead of serving.
"""
from __future__ import annotations

import logging
import os
from typing import Optional

import torch

log = logging.getLogger("sdcguard")


class RequirementNotMet(RuntimeError):
    """SDCGUARD_REQUIRE is set and the server would run unchecked."""


class _Plugin:
    """What register() installs: the wrapped methods, one ServeGuard per device, the layers' selection order."""

    def __init__(self, z: float, share: float, offset: int):
        self.z, self.share, self.offset = z, share, offset
        self.guards: dict = {}
        self.loaded = 0                  # eligible layers seen, in load order (a reload keeps a layer's number)

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
    plugin = _PLUGIN[0] = _Plugin(z, share, int(_float_env("SDCGUARD_OFFSET", 0)))

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
    for g in p.guards.values():
        g.detach()


def plugin_state() -> Optional[_Plugin]:
    return _PLUGIN[0]
