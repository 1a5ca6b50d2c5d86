"""EchoKV settings from ``ECHOKV_*`` environment variables.

The variables, their defaults, their meaning and the ``ValueError`` a bad value
raises are those of ``echokv_vllm/config.py:40-99``:

    ECHOKV_ENABLE           1 to install the backend (plugin.register)
    ECHOKV_FIXED_BITS       pin every layer to this tier (controller off)
    ECHOKV_MEM_BITS         memory budget, bits/element: 2, 4, 6 or 8 (default 4, or
                            what ECHOKV_FIXED_BITS needs when that is set)
    ECHOKV_INIT_BITS        starting tier (default: highest tier the budget gives
                            every block: 8, 4, 4, 2 for budgets 8, 6, 4, 2)
    ECHOKV_FROZEN           1 to keep tiers fixed while the canary keeps measuring
    ECHOKV_TAU0             per-layer canary KL budget (default 0.01)
    ECHOKV_L0               reference context length for tau scaling (default 4096)
    ECHOKV_TAU_SCALING      none (default) or sqrt
    ECHOKV_ALPHA            EMA weight of the newest sample (default 0.1)
    ECHOKV_K_GROUP          tokens per per-channel K group (default 32; power of 2, >= 16)
    ECHOKV_V_GROUP          head_dim elements per per-token V group (default 32)
    ECHOKV_RESIDUAL_SLOTS   open-K-group slots per layer (default max_num_seqs + 16)
    ECHOKV_CANARY_INTERVAL  fire every N model steps, all layers together (default 64)
    ECHOKV_KREF_WINDOW      K_ref ring size in tokens (default 64; >= ECHOKV_K_GROUP)
    ECHOKV_CANARY_MAX_Q     decode queries sampled per fire (default 8)

This build's own: ECHOKV_OWN_GROUP_EXACT=1 (prefill sees each query's own K
group at full precision) and ECHOKV_BATCH_INVARIANT=0 (the balanced decode
schedule); ECHOKV_V_GROUP is 1 to 256 channels.

Read elsewhere: ECHOKV_CUDAGRAPH=0 keeps attention out of full graphs (the
backend), ECHOKV_CHECK_HOST_SLOTS=1 checks the host slot mapping every step. The
reference's Triton-only switches (ECHOKV_DISABLE_TRITON, ECHOKV_AUTOTUNE,
ECHOKV_PREFILL_ROWS) have no meaning here and are ignored.

Each setting is one row of ``SETTINGS``: its variable, how to parse it, its
default (a function of the settings resolved before it) and its check. Rows are
resolved in order, then checked in order, so the first bad value raises.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Any, Callable, NamedTuple

from echokv_amd.controller import SUPPORTED_BITS, ControllerParams


@dataclass(frozen=True)
class EchoKVConfig:
    mem_bits: int = 4
    k_group: int = 32
    v_group: int = 32
    residual_slots: int | None = None
    canary_interval: int = 64
    kref_window: int = 64
    canary_max_q: int = 8
    own_group_exact: bool = False
    batch_invariant: bool = True
    controller: ControllerParams = field(default_factory=ControllerParams)


def default_init_bits(mem_bits: int) -> int:
    """The highest tier every block can hold under a ``mem_bits`` budget."""
    fits = [b for b in SUPPORTED_BITS if b <= mem_bits]
    return fits[-1] if fits else 2


def _flag(raw: str) -> bool:
    return raw == "1"


def _tier(name: str):
    def check(v, _):
        if v is not None and v not in SUPPORTED_BITS:
            return f"{name} must be one of {SUPPORTED_BITS}, got {v}"
    return check


def _is_pow2(x: int) -> bool:
    return x > 0 and not x & (x - 1)


def v_group_supported(v_group: int, head_size: int | None = None) -> bool:
    """V groups the kernels store and read: 1 to 256 channels, dividing the head
    size when one is given (the reference's rule, ``backend.py:100-102``)."""
    return 1 <= v_group <= 256 and (head_size is None or head_size % v_group == 0)


class Setting(NamedTuple):
    env: str
    key: str
    parse: Callable[[str], Any]
    default: Callable[[dict], Any]
    check: Callable[[Any, dict], str | None] | None = None


SETTINGS: tuple[Setting, ...] = (
    Setting("ECHOKV_FIXED_BITS", "fixed_bits", int, lambda s: None, _tier("ECHOKV_FIXED_BITS")),
    # A pinned tier with no explicit budget gets a budget that holds it.
    Setting("ECHOKV_MEM_BITS", "mem_bits", int, lambda s: 4 if s["fixed_bits"] is None else max(s["fixed_bits"], 2),
            lambda v, s: None if v in (2, 4, 6, 8) else f"ECHOKV_MEM_BITS must be 2, 4, 6 or 8, got {v}"),
    Setting("ECHOKV_INIT_BITS", "init_bits", int, lambda s: default_init_bits(s["mem_bits"]),
            _tier("ECHOKV_INIT_BITS")),
    Setting("ECHOKV_FROZEN", "frozen", _flag, lambda s: False),
    Setting("ECHOKV_TAU0", "tau0", float, lambda s: 0.01),
    Setting("ECHOKV_L0", "l0", int, lambda s: 4096),
    Setting("ECHOKV_TAU_SCALING", "tau_scaling", str, lambda s: "none",
            lambda v, s: None if v in ("none", "sqrt") else "ECHOKV_TAU_SCALING must be none or sqrt"),
    Setting("ECHOKV_ALPHA", "alpha", float, lambda s: 0.1),
    Setting("ECHOKV_K_GROUP", "k_group", int, lambda s: 32,
            lambda v, s: None if v >= 16 and _is_pow2(v) else f"ECHOKV_K_GROUP must be a power of 2 and >= 16, got {v}"),
    # Any V group that divides the head size, as the reference (checked against the
    # head size in supports_head_size and TieredLayout).
    Setting("ECHOKV_V_GROUP", "v_group", int, lambda s: 32,
            lambda v, s: None if v_group_supported(v) else
            f"ECHOKV_V_GROUP must be 1 to 256 channels, got {v}"),
    Setting("ECHOKV_RESIDUAL_SLOTS", "residual_slots", int, lambda s: None),
    Setting("ECHOKV_CANARY_INTERVAL", "canary_interval", int, lambda s: 64,
            lambda v, s: None if v >= 1 else "ECHOKV_CANARY_INTERVAL must be >= 1"),
    Setting("ECHOKV_KREF_WINDOW", "kref_window", int, lambda s: 64,
            lambda v, s: None if v >= s["k_group"] else "ECHOKV_KREF_WINDOW must be >= ECHOKV_K_GROUP"),
    Setting("ECHOKV_CANARY_MAX_Q", "canary_max_q", int, lambda s: 8),
    # This build's own (no reference counterpart): prefill sees each query's own K group
    # at full precision, as decode did (the fix docs/ECHOKV_VLLM_PLUGIN.md:261-266 names).
    Setting("ECHOKV_OWN_GROUP_EXACT", "own_group_exact", _flag, lambda s: False,
            lambda v, s: None if not v or s["k_group"] <= 64 else "ECHOKV_OWN_GROUP_EXACT needs ECHOKV_K_GROUP <= 64"),
    # This build's own: 1 (default) splits each decode sequence by its own length, so
    # its result does not depend on the batch (the reference's decode semantics); 0
    # spreads the batch's blocks evenly over the GPU (faster on uneven batches).
    Setting("ECHOKV_BATCH_INVARIANT", "batch_invariant", lambda raw: raw != "0", lambda s: True),
)

_CONTROLLER_KEYS = ("tau0", "l0", "tau_scaling", "alpha", "init_bits", "fixed_bits", "frozen")


def resolve(environ=None) -> dict:
    """Every setting's value (parsed, or its default), after all checks pass."""
    env = os.environ if environ is None else environ
    vals: dict = {}
    for st in SETTINGS:
        raw = env.get(st.env)
        vals[st.key] = st.default(vals) if raw is None or raw == "" else st.parse(raw)
    for st in SETTINGS:
        if st.check is not None and (msg := st.check(vals[st.key], vals)):
            raise ValueError(msg)
    return vals


def load_config(environ=None) -> EchoKVConfig:
    vals = resolve(environ)
    ctrl = ControllerParams(**{k: vals[k] for k in _CONTROLLER_KEYS})
    return EchoKVConfig(controller=ctrl, **{k: vals[k] for k in vals if k not in _CONTROLLER_KEYS})
