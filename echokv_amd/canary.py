"""Absolute canary: full-precision K_ref ring + per-tier attention KL.

Interface of ``echokv_vllm/canary.py`` (``ring_view`` 19-23, ``KRefRing``
26-56, ``canary_kl`` 59-89):

    δ̂_b = KL( softmax(Q · K̃_bᵀ · s) ‖ softmax(Q · K_refᵀ · s) ),  K̃_b = storage round trip of K_ref at b bits

K_ref holds the most recent keys in float32, captured before they are
quantized, so the probe never reads the cache. ``canary_kl`` is one HIP launch
per call (``echokv_amd/csrc/canary.hip``): every (layer, KV head) pair is a
workgroup, for all layers at once.

A ring of ``W`` slots with ``fill`` valid keys and next write position ``pos``
holds key ``i`` (oldest first) in slot ``(pos - fill + i) mod W``: the view is
one gather by that index, a push one scatter.
"""

from __future__ import annotations

import torch

from echokv_amd import _lib


def _ring_index(size: int, pos: int, fill: int, device) -> torch.Tensor:
    return (torch.arange(fill, device=device) + (pos - fill)) % size


def ring_view(buf: torch.Tensor, pos: int, fill: int, dim: int = 0) -> torch.Tensor:
    """The ``fill`` keys of a ring buffer along ``dim``, oldest first (``pos`` = next write)."""
    size = buf.shape[dim]
    if not 0 <= fill <= size:
        raise ValueError(f"ring of {size} slots cannot hold {fill} keys")
    if fill < size and pos == fill:  # never wrapped: the keys are the leading slots
        return buf.narrow(dim, 0, fill)
    return buf.index_select(dim, _ring_index(size, pos, fill, buf.device))


class KRefRing:
    """Circular buffer of the last ``window`` keys, ``[window, H, D]`` float32."""

    def __init__(self, window: int) -> None:
        if window < 2:
            raise ValueError("K_ref window must be >= 2")
        self.window = window
        self.buf: torch.Tensor | None = None
        self.fill = 0
        self.pos = 0

    def push(self, keys: torch.Tensor) -> None:
        """Append ``keys [t, H, D]`` (only the newest ``window`` of them can stay)."""
        t = min(keys.shape[0], self.window)
        if t == 0:
            return
        keys = keys[keys.shape[0] - t :].float()
        if self.buf is None:
            self.buf = torch.zeros(self.window, *keys.shape[1:], device=keys.device)
        slots = (torch.arange(t, device=keys.device) + self.pos) % self.window
        self.buf.index_copy_(0, slots, keys)
        self.pos = (self.pos + t) % self.window
        self.fill = min(self.window, self.fill + t)

    def view(self) -> torch.Tensor | None:
        if self.buf is None or self.fill < 2:
            return None
        return ring_view(self.buf, self.pos, self.fill)


def canary_kl(query: torch.Tensor, kref: torch.Tensor, bits: tuple, k_group: int, softmax_scale: float,
              out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Mean per-head, per-query KL at each tier in ``bits``; float32 ``[..., len(bits)]``.

    query ``[..., nq, Hq, D]``; kref ``[..., W, H, D]`` oldest first; leading dims
    (e.g. layers) are independent problems. Only whole ``k_group`` groups of
    K_ref are scored (the oldest ``W mod k_group`` keys are dropped).
    ``workspace``: float32 with at least layers * H * len(bits) elements."""
    w = (kref.shape[-3] // k_group) * k_group
    if w == 0:
        raise ValueError(f"K_ref has {kref.shape[-3]} keys, fewer than k_group={k_group}")
    _lib.require_device(query, kref)
    lead = query.shape[:-3]
    nq, hq, d = query.shape[-3:]
    q = query.reshape(-1, nq, hq, d)
    k = kref.float().reshape(-1, *kref.shape[-3:])
    if q.stride(3) != 1:
        q = q.contiguous()
    if k.stride(3) != 1:
        k = k.contiguous()
    layers, h = q.shape[0], k.shape[2]
    if k.shape[0] != layers:
        raise ValueError("query and kref must share their leading dims")
    packed = 0
    for i, b in enumerate(bits):
        packed |= int(b) << (8 * i)
    if out is None:
        out = torch.empty(layers, len(bits), device=query.device, dtype=torch.float32)
    if workspace is None:
        workspace = torch.empty(layers * h * len(bits), device=query.device, dtype=torch.float32)
    elif workspace.dtype != torch.float32 or workspace.numel() < layers * h * len(bits):
        raise ValueError("canary workspace is too small")
    _lib.call(
        "echokv_canary_kl", _lib.ptr(q), _lib.dtype_code(q), q.stride(0), q.stride(1), q.stride(2),
        _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2), layers, nq, hq, h, d, k.shape[1],
        len(bits), packed, k_group, float(softmax_scale), _lib.ptr(workspace), _lib.ptr(out), _lib.stream(),
    )
    return out.reshape(*lead, len(bits))
