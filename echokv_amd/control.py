"""Inspect and steer EchoKV layers inside a running engine.

Interface of ``echokv_vllm/control.py:39-117``. Every function takes the model as
its first argument, so vLLM can ship it to every worker with
``llm.apply_model(fn)`` (``functools.partial`` for the other arguments; vLLM
needs ``VLLM_ALLOW_INSECURE_SERIALIZATION=1`` for that)::

    from functools import partial
    from echokv_amd import control
    llm.apply_model(partial(control.set_tier_vector, bits=[4] * 32))
    state = llm.apply_model(control.get_state)[0]   # rank 0
"""

from __future__ import annotations

import re

import torch

from echokv_amd.backend import EchoKVAttentionImpl
from echokv_amd.controller import SUPPORTED_BITS

_LAYER_NUMBER = re.compile(r"layers\.(\d+)\.")


def iter_layers(model: torch.nn.Module):
    """(layer_name, impl) of every EchoKV attention layer, in layer order (the
    number in ``layers.<n>.`` of the name; modules without one keep their order)."""
    found = []
    for name, mod in model.named_modules():
        impl = getattr(mod, "impl", None)
        if isinstance(impl, EchoKVAttentionImpl):
            layer_name = getattr(mod, "layer_name", name)
            m = _LAYER_NUMBER.search(layer_name)
            found.append((int(m.group(1)) if m else len(found), layer_name, impl))
    found.sort(key=lambda x: x[0])
    return [(layer_name, impl) for _, layer_name, impl in found]


def _by_tier(d: dict) -> dict:
    return {str(b): v for b, v in d.items()}


def get_state(model: torch.nn.Module) -> dict:
    """Per-layer tier, canary EMAs, fire / transition counts and storage counters,
    plus the tier vector and the model-wide stored bits per element."""
    layers = []
    written = dict.fromkeys(SUPPORTED_BITS, 0)
    for name, impl in iter_layers(model):
        c = impl.controller
        entry = {"layer": name, "bits": c.bits, "ema": _by_tier(c.ema), "fires": c.fires,
                 "transitions": c.transitions, "forward_calls": impl.forward_calls}
        s = impl.store
        if s is not None:
            tw = s.tokens_written
            entry.update(tokens_written=_by_tier(tw), blocks_opened=_by_tier(s.blocks_opened),
                         downgraded_blocks=s.downgraded_blocks, demoted_blocks=s.demoted_blocks,
                         sealed_groups=s.sealed_groups, pool_free=s.pool_free, pool_size=s.pool_size)
            for b, v in tw.items():
                written[b] += v
        layers.append(entry)
    total = sum(written.values())
    return {"tier_vector": [e["bits"] for e in layers], "tokens_written": _by_tier(written),
            "avg_stored_bits": sum(b * v for b, v in written.items()) / total if total else None, "layers": layers}


def get_tier_vector(model: torch.nn.Module) -> list[int]:
    return [impl.controller.bits for _, impl in iter_layers(model)]


def set_tier_vector(model: torch.nn.Module, bits) -> int:
    """Set each layer's tier (an int sets every layer). Blocks opened from now on
    take it; blocks already open keep theirs. Returns the number of layers."""
    layers = iter_layers(model)
    vec = [bits] * len(layers) if isinstance(bits, int) else list(bits)
    if len(vec) != len(layers):
        raise ValueError(f"got {len(vec)} tiers for {len(layers)} layers")
    bad = [b for b in vec if b not in SUPPORTED_BITS]
    if bad:
        raise ValueError(f"unsupported tier {bad[0]}")
    for (_, impl), b in zip(layers, vec):
        impl.controller.bits = b
    return len(layers)


def _set_param(model: torch.nn.Module, name: str, value) -> int:
    layers = iter_layers(model)
    for _, impl in layers:
        setattr(impl.controller.params, name, value)
    return len(layers)


def set_frozen(model: torch.nn.Module, frozen: bool) -> int:
    """Stop (or resume) tier changes; the canary keeps updating the EMAs."""
    return _set_param(model, "frozen", bool(frozen))


def set_tau0(model: torch.nn.Module, tau0: float) -> int:
    return _set_param(model, "tau0", float(tau0))


def reset_counters(model: torch.nn.Module) -> int:
    """Zero the storage counters and forward-call counts (e.g. between warm-up and measurement)."""
    layers = iter_layers(model)
    for _, impl in layers:
        if impl.store is not None:
            impl.store.reset_counters()
        impl.forward_calls = 0
    return len(layers)
