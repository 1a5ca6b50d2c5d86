"""The canary's per-tier attention KL (oracle; test infrastructure only).

Restates ``echokv_vllm/canary.py:59-89``: for each tier b, K~_b is the
per-channel storage round trip of the K_ref keys over whole ``k_group``
groups (the oldest ``W mod k_group`` keys are dropped), and
δ_b = mean over query rows and heads of KL(softmax(q·K~_bᵀ·s) ‖ softmax(q·K_refᵀ·s)),
clamped at zero. Inputs are oldest-first (``canary.py:19-23`` rolls a ring).
"""

from __future__ import annotations

import numpy as np

from oracle.quant import fake_quant_channels


def _log_softmax(x):
    m = x.max(axis=-1, keepdims=True)
    y = x - m
    return y - np.log(np.exp(y).sum(axis=-1, keepdims=True))


def canary_kl(query, kref, bits, k_group, scale):
    """query ``[..., nq, Hq, D]``, kref ``[..., W, H, D]`` -> ``[..., len(bits)]`` float32."""
    w = (kref.shape[-3] // k_group) * k_group
    if w == 0:
        raise ValueError(f"K_ref has {kref.shape[-3]} keys, fewer than k_group={k_group}")
    kref = kref[..., kref.shape[-3] - w :, :, :].astype(np.float32)
    q = np.swapaxes(query.astype(np.float64), -3, -2)  # [..., Hq, nq, D]
    rep = q.shape[-3] // kref.shape[-2]

    def logw(k):
        kh = np.repeat(np.swapaxes(k.astype(np.float64), -3, -2), rep, axis=-3)  # [..., Hq, W, D]
        return _log_softmax(q @ np.swapaxes(kh, -1, -2) * scale)

    lref = logw(kref)
    out = []
    for b in bits:
        lq = logw(fake_quant_channels(kref, b, k_group))
        out.append((np.exp(lq) * (lq - lref)).sum(-1).mean(axis=(-2, -1)))
    return np.maximum(np.stack(out, -1), 0.0).astype(np.float32)
