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


_MANTISSA = {torch.float16: (10, -14), torch.bfloat16: (7, -126)}  # mantissa bits, min normal exponent


def half_ulp(ref, dtype) -> np.ndarray:
    """Half the spacing of ``dtype`` at each reference value: the rounding error
    an output stored in that dtype carries however exact the kernel is."""
    if dtype not in _MANTISSA:
        return np.zeros(np.shape(ref))
    mant, emin = _MANTISSA[dtype]
    a = np.abs(np.asarray(ref, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** emin)))  # subnormals share the min-normal spacing
    return np.exp2(e - mant) / 2


def maxdiff(got, ref) -> float:
    """Max |got - ref| over elements; for an fp16 / bf16 output, beyond half the
    output dtype's spacing at ref, so storing the dtype's neighbour of an exact
    result is not counted against the kernel and anything more is."""
    ref = np.asarray(ref, np.float64)
    if torch.is_tensor(got):
        slack = half_ulp(ref, got.dtype)
        g = got.detach().float().cpu().numpy().astype(np.float64)
    else:
        slack, g = 0.0, np.asarray(got, np.float64)
    return float((np.abs(g - ref) - slack).max())
