"""Helpers of the GPU parity tests: replay a write script through the product's
``TieredKVCache`` on the device, and move arrays between numpy and torch."""

from __future__ import annotations

import numpy as np
import torch

import scripts as S
from echokv_amd.tiered_cache import TieredKVCache, TieredLayout


def gpu_store(s, device):
    layout = TieredLayout(s.h, s.d, s.bs, s.mem_bits, s.kg, s.vg)
    page = s.bs * TieredLayout.per_token_bytes(s.h, s.d, s.mem_bits, s.kg, s.vg)
    stride = page + s.row_pad
    backing = torch.full((s.num_blocks * stride + 64,), 0xAB, dtype=torch.uint8, device=device)
    pages = torch.as_strided(backing, (s.num_blocks, page), (stride, 1))
    rdt = torch.float16 if s.dtype == "f16" else torch.float32
    store = TieredKVCache(layout, pages, residual_slots=s.residual_slots, residual_dtype=rdt)
    return store, backing, stride, page


def gpu_replay(s, device):
    """(store, backing, stride, page, kref) after every step of ``s``."""
    store, backing, stride, page = gpu_store(s, device)
    kref = None if s.kref_window is None else torch.zeros(s.kref_window, s.h, s.d, device=device)
    for slots, bits, k, v in S.script_inputs(s):
        store.write(torch.from_numpy(k).to(device), torch.from_numpy(v).to(device),
                    torch.from_numpy(slots).to(device), bits, kref=kref)
    torch.cuda.synchronize()
    return store, backing, stride, page, kref


def t(a, device, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return x if dtype is None else x.to(dtype)


def maxdiff(got, ref) -> float:
    g = got.detach().float().cpu().numpy() if torch.is_tensor(got) else np.asarray(got, np.float64)
    return float(np.abs(g.astype(np.float64) - np.asarray(ref, np.float64)).max())
