"""Per-layer tier controller: EMA of the canary's δ̂ per tier, lowest tier under τ.

Interface and rule of ``echokv_vllm/controller.py:11-68``: every canary fire
updates ``ema[b]`` (α-weighted) for every tier; unless frozen or pinned the
layer moves to the lowest tier whose EMA is below τ, else the highest tier.
With ``tau_scaling="sqrt"``, τ(L) = τ0·sqrt(max(L, L0)/L0).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

SUPPORTED_BITS = (2, 4, 8)


@dataclass
class ControllerParams:
    tau0: float = 0.01
    l0: int = 4096
    tau_scaling: str = "none"
    alpha: float = 0.1
    init_bits: int = 8
    fixed_bits: int | None = None
    frozen: bool = False


@dataclass
class LayerController:
    params: ControllerParams
    bits: int = 0
    ema: dict = field(default_factory=lambda: {b: None for b in SUPPORTED_BITS})
    fires: int = 0
    transitions: int = 0

    def __post_init__(self) -> None:
        if not self.bits:
            self.bits = self.params.fixed_bits or self.params.init_bits

    def tau(self, ctx_len: float) -> float:
        p = self.params
        if p.tau_scaling == "sqrt":
            return p.tau0 * math.sqrt(max(ctx_len, p.l0) / p.l0)
        return p.tau0

    def observe(self, deltas: dict, ctx_len: float) -> None:
        a = self.params.alpha
        for b, d in deltas.items():
            prev = self.ema[b]
            self.ema[b] = d if prev is None else a * d + (1.0 - a) * prev
        self.fires += 1
        if self.params.frozen or self.params.fixed_bits is not None:
            return
        tau = self.tau(ctx_len)
        new = next((b for b in sorted(SUPPORTED_BITS) if self.ema[b] is not None and self.ema[b] < tau),
                   max(SUPPORTED_BITS))
        if new != self.bits:
            self.transitions += 1
            self.bits = new
