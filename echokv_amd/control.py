"""Inspect and steer EchoKV layers inside a running engine.

Interface of ``echokv_vllm/control.py:39-117``: the function names, their
arguments and return values, and the keys of ``get_state``. Every function
takes the model first, so vLLM can run it on every worker with
``llm.apply_model(fn)`` (``functools.partial`` binds the other arguments; vLLM
needs ``VLLM_ALLOW_INSECURE_SERIALIZATION=1`` to ship a partial)::

    from functools import partial
    from echokv_vllm import control
    llm.apply_model(partial(control.set_tier_vector, bits=[4] * 32))
    state = llm.apply_model(control.get_state)[0]   # rank 0

Layers are the modules whose ``impl`` is an ``EchoKVAttentionImpl``, in model
order: sorted by the numbers in their layer names read as integers (so
``layers.10`` follows ``layers.9``), ties in the order ``named_modules`` gives;
names without a number come first.
"""

from __future__ import annotations

import re

import torch

from echokv_amd.backend import EchoKVAttentionImpl
from echokv_amd.controller import SUPPORTED_BITS

_DIGITS = re.compile(r"(\d+)")


def _model_order(name: str, seen: int) -> tuple:
    """Sort key: the name's runs of digits as integers, then discovery order."""
    return tuple(int(part) for part in _DIGITS.findall(name)), seen


def iter_layers(model: torch.nn.Module) -> list:
    """``(layer_name, impl)`` of every EchoKV attention layer, in model order."""
    layers = []
    for path, module in model.named_modules():
        impl = getattr(module, "impl", None)
        if isinstance(impl, EchoKVAttentionImpl):
            name = getattr(module, "layer_name", path)
            layers.append((_model_order(name, len(layers)), name, impl))
    return [(name, impl) for _, name, impl in sorted(layers, key=lambda x: x[0])]


def _per_tier(values: dict) -> dict:
    """Tier-keyed counters with string keys (the JSON form ``get_state`` returns)."""
    return {str(b): values[b] for b in SUPPORTED_BITS if b in values}


def _layer_state(name: str, impl: EchoKVAttentionImpl) -> dict:
    ctl = impl.controller
    state = {"layer": name, "bits": ctl.bits, "ema": _per_tier(ctl.ema), "fires": ctl.fires,
             "transitions": ctl.transitions, "forward_calls": impl.forward_calls}
    store = impl.store
    if store is not None:  # bound to a KV cache: the storage counters too
        state["tokens_written"] = _per_tier(store.tokens_written)
        state["blocks_opened"] = _per_tier(store.blocks_opened)
        for key in ("downgraded_blocks", "demoted_blocks", "sealed_groups", "pool_free", "pool_size"):
            state[key] = getattr(store, key)
    return state


def get_state(model: torch.nn.Module) -> dict:
    """Per-layer tier, canary EMAs, fire / transition counts and storage counters,
    the tier vector, the model-wide tokens written per tier and the stored bits per
    element they average to (None before anything is written)."""
    layers = [_layer_state(name, impl) for name, impl in iter_layers(model)]
    totals = {b: sum(int(s.get("tokens_written", {}).get(str(b), 0)) for s in layers) for b in SUPPORTED_BITS}
    count = sum(totals.values())
    return {
        "tier_vector": [s["bits"] for s in layers],
        "tokens_written": _per_tier(totals),
        "avg_stored_bits": sum(b * n for b, n in totals.items()) / count if count else None,
        "layers": layers,
    }


def get_tier_vector(model: torch.nn.Module) -> list[int]:
    return [impl.controller.bits for _, impl in iter_layers(model)]


def set_tier_vector(model: torch.nn.Module, bits) -> int:
    """Set each layer's tier (one int sets every layer). Blocks opened from now on
    take it; blocks already open keep theirs. Returns the number of layers; raises
    ``ValueError`` (changing nothing) for a wrong length or an unsupported tier."""
    impls = [impl for _, impl in iter_layers(model)]
    tiers = [bits] * len(impls) if isinstance(bits, int) else list(bits)
    if len(tiers) != len(impls):
        raise ValueError(f"got {len(tiers)} tiers for {len(impls)} layers")
    unsupported = sorted({b for b in tiers if b not in SUPPORTED_BITS})
    if unsupported:
        raise ValueError(f"unsupported tier {unsupported[0]} (tiers are {SUPPORTED_BITS})")
    for impl, b in zip(impls, tiers):
        impl.controller.bits = b
    return len(impls)


def _for_each_controller(model: torch.nn.Module, **params) -> int:
    impls = [impl for _, impl in iter_layers(model)]
    for impl in impls:
        for key, value in params.items():
            setattr(impl.controller.params, key, value)
    return len(impls)


def set_frozen(model: torch.nn.Module, frozen: bool) -> int:
    """Stop (or resume) tier changes; the canary keeps updating the EMAs."""
    return _for_each_controller(model, frozen=bool(frozen))


def set_tau0(model: torch.nn.Module, tau0: float) -> int:
    """Set every layer's canary KL budget."""
    return _for_each_controller(model, tau0=float(tau0))


def reset_counters(model: torch.nn.Module) -> int:
    """Zero the storage counters and forward-call counts (e.g. between warm-up and measurement)."""
    layers = iter_layers(model)
    for _, impl in layers:
        impl.forward_calls = 0
        if impl.store is not None:
            impl.store.reset_counters()
    return len(layers)
