"""Small host helpers (``echokv_vllm/_util.py:8-20``)."""

from __future__ import annotations

import torch


def to_device(t: torch.Tensor, device) -> torch.Tensor:
    """Host tensor -> ``device`` without blocking the CPU: a pinned staging copy and a
    non-blocking transfer, so the host keeps planning while the GPU runs."""
    device = torch.device(device)
    if device.type != "cuda":
        return t.to(device)
    return t.pin_memory().to(device, non_blocking=True)
