"""Storage numerics in numpy (oracle; test infrastructure only).

Restates ``echokv_vllm/quant.py:22-120``: group-asymmetric quantization with
an fp16 scale and an fp16 *float* minimum, both rounded to fp16 before the
codes are computed. All arithmetic is IEEE float32 (correctly rounded
subtraction and division), codes round half to even, fp16 casts are RNE.
"""

from __future__ import annotations

import numpy as np

SUPPORTED_BITS = (2, 4, 8)  # quant.py:22
FP16_TINY = np.float32(2.0 ** -14)  # quant.py:23, smallest normal fp16


def _levels(bits: int) -> np.float32:
    return np.float32((1 << bits) - 1)


def quantize(x: np.ndarray, bits: int, group_size: int):
    """quant.py:26-45. Returns (codes u8 [..., D], scale f16 [..., G], min f16 [..., G])."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"unsupported bits: {bits}")
    d = x.shape[-1]
    if d % group_size:
        raise ValueError(f"head dim {d} not divisible by group_size {group_size}")
    xg = x.astype(np.float32).reshape(*x.shape[:-1], d // group_size, group_size)
    mn16 = xg.min(axis=-1).astype(np.float16)
    mn = mn16.astype(np.float32)
    scale16 = np.maximum((xg.max(axis=-1) - mn) / _levels(bits), FP16_TINY).astype(np.float16)
    q = np.rint((xg - mn[..., None]) / scale16.astype(np.float32)[..., None])
    q = np.clip(q, 0, _levels(bits))
    return q.reshape(x.shape).astype(np.uint8), scale16, mn16


def dequantize(codes, scale, mn, group_size: int) -> np.ndarray:
    """quant.py:48-55: code * scale + min in float32 (the product is exact)."""
    d = codes.shape[-1]
    qg = codes.astype(np.float32).reshape(*codes.shape[:-1], d // group_size, group_size)
    out = qg * scale.astype(np.float32)[..., None] + mn.astype(np.float32)[..., None]
    return out.reshape(codes.shape)


def fake_quant(x, bits: int, group_size: int) -> np.ndarray:
    """quant.py:58-60."""
    return dequantize(*quantize(x, bits, group_size), group_size)


def stats_along(x, bits: int, axis: int):
    """quant.py:63-69: fp16 (scale, min) of ``x`` reduced over ``axis``."""
    xf = x.astype(np.float32)
    mn16 = xf.min(axis=axis).astype(np.float16)
    scale16 = np.maximum((xf.max(axis=axis) - mn16.astype(np.float32)) / _levels(bits), FP16_TINY).astype(np.float16)
    return scale16, mn16


def quantize_with(x, scale, mn, bits: int) -> np.ndarray:
    """quant.py:72-75: codes under given fp16 stats (clamped)."""
    q = np.rint((x.astype(np.float32) - mn.astype(np.float32)) / scale.astype(np.float32))
    return np.clip(q, 0, _levels(bits)).astype(np.uint8)


def dequantize_with(codes, scale, mn) -> np.ndarray:
    """quant.py:78-79."""
    return codes.astype(np.float32) * scale.astype(np.float32) + mn.astype(np.float32)


def fake_quant_channels(k, bits: int, group: int) -> np.ndarray:
    """quant.py:82-96: per-channel round trip over consecutive ``group``-token groups
    of ``k [..., T, H, D]``; a trailing partial group stays exact."""
    t = k.shape[-3]
    full = (t // group) * group
    out = k.astype(np.float32).copy()
    if full:
        kg = out[..., :full, :, :].reshape(*k.shape[:-3], full // group, group, *k.shape[-2:])
        scale, mn = stats_along(kg, bits, axis=-3)
        codes = quantize_with(kg, scale[..., None, :, :], mn[..., None, :, :], bits)
        deq = dequantize_with(codes, scale[..., None, :, :], mn[..., None, :, :])
        out[..., :full, :, :] = deq.reshape(*k.shape[:-3], full, *k.shape[-2:])
    return out


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """quant.py:99-110: little-endian inside a byte (element i at bits [i*b, (i+1)*b))."""
    if bits == 8:
        return codes.astype(np.uint8)
    per = 8 // bits
    c = codes.reshape(*codes.shape[:-1], codes.shape[-1] // per, per).astype(np.uint32)
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    return (c << shifts).sum(axis=-1).astype(np.uint8)


def unpack(packed: np.ndarray, bits: int) -> np.ndarray:
    """quant.py:113-120."""
    if bits == 8:
        return packed.astype(np.uint8)
    per = 8 // bits
    shifts = np.arange(per, dtype=np.uint32) * bits
    c = (packed.astype(np.uint32)[..., None] >> shifts) & ((1 << bits) - 1)
    return c.reshape(*packed.shape[:-1], packed.shape[-1] * per).astype(np.uint8)
