"""Quantize-on-write entry points (``echokv_vllm/kernels/write.py:29-50``).

``write_tokens`` stores every token row of a step in one launch (V per token,
K to the residual / under sealed stats / into the K_ref ring); ``finalize_k``
quantizes each completed K group per channel; ``write_step`` is the pair as one
launch (the store's per-step path). Both read each block's tier
from its page header on the device and everything else from ``WriteMeta``,
so one launch covers INT2/INT4/INT8 blocks and a HIP graph can capture them.
Kernels: ``echokv_amd/csrc/store.hip`` via ``echokv_write_tokens`` /
``echokv_finalize_k`` / ``echokv_write_step``.
"""

from __future__ import annotations

import torch

from echokv_amd import _lib


def _kv(t: torch.Tensor, n_rows: int) -> torch.Tensor:
    """``t`` with contiguous channels; every one of the step's ``n_rows`` rows is
    read (a row's words are requested before its slot is known)."""
    if t.shape[0] < n_rows:
        raise ValueError(f"key / value hold {t.shape[0]} rows, the step has {n_rows} token rows")
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def write_tokens(store, key: torch.Tensor, value: torch.Tensor, meta, kref: torch.Tensor | None = None) -> None:
    """Store the ``meta.n_rows`` token rows of ``key``/``value`` ``[T, H, D]`` as ``meta.tok`` says."""
    if meta.n_rows == 0:
        return
    _lib.require_device(key, value, store.pages)
    key, value = _kv(key, meta.n_rows), _kv(value, meta.n_rows)
    if value.dtype != key.dtype:
        value = value.to(key.dtype)
    tok = meta.tok
    if tok.stride(1) != 1 or tok.dtype != torch.int64:
        raise ValueError("meta.tok must be int64 with contiguous rows")
    kref, ks0, ks1 = _kref_args(store, kref)
    res = _lib.residual(store.res_k)
    _lib.call(
        "echokv_write_tokens", _lib.byref(store.abi), _lib.ptr(store.pages),
        _lib.ptr(key), key.stride(0), key.stride(1), _lib.ptr(value), value.stride(0), value.stride(1),
        _lib.dtype_code(key), _lib.ptr(tok), tok.stride(0), meta.n_rows, _lib.byref(res),
        _lib.ptr(kref), ks0, ks1, _lib.stream(),
    )


def _fin_rows(store, meta):
    fin = meta.fin
    width = 3 + store.layout.k_group
    if fin.dtype != torch.int64 or fin.shape[-1] != width or fin.stride(1) != 1 or fin.stride(0) != width:
        raise ValueError(f"meta.fin must be int64 [n, {width}] with contiguous rows (row stride {width})")
    return fin


def _kref_args(store, kref):
    if kref is None:
        return None, 0, 0
    if kref.dtype != torch.float32 or kref.stride(2) != 1:
        raise ValueError("the K_ref ring must be float32 with contiguous rows")
    if kref.shape[0] < store.planner.kref_window:
        raise ValueError(f"the K_ref ring has {kref.shape[0]} rows, the planner writes {store.planner.kref_window}")
    return kref, kref.stride(0), kref.stride(1)


FUSED_MAX_K_GROUP = 256


def write_step(store, key: torch.Tensor, value: torch.Tensor, meta, kref: torch.Tensor | None = None,
               full_grid: bool = False) -> None:
    """``finalize_k`` then ``write_tokens`` of one step, as one launch (same results).

    ``full_grid`` gives the finalize part one workgroup per token row, masked on
    the device by ``meta.fin_count`` (a captured graph does not know the count)."""
    n_fin = meta.n_rows if full_grid else meta.n_fin
    # The kernel reads every fin row below its grid (the device count masks them),
    # and the staged rows cover the count: the grid stops at the rows there are.
    n_fin = min(n_fin, meta.fin.shape[0])
    if n_fin + meta.n_rows == 0:
        return
    if store.layout.k_group > FUSED_MAX_K_GROUP:
        raise ValueError(f"the fused step takes k_group <= {FUSED_MAX_K_GROUP}, got {store.layout.k_group}")
    fin = _fin_rows(store, meta)  # rows at or past the device count are never read
    _lib.require_device(key, value, store.pages)
    key, value = _kv(key, meta.n_rows), _kv(value, meta.n_rows)
    if value.dtype != key.dtype:
        value = value.to(key.dtype)
    tok = meta.tok
    if tok.stride(1) != 1 or tok.dtype != torch.int64:
        raise ValueError("meta.tok must be int64 with contiguous rows")
    kref, ks0, ks1 = _kref_args(store, kref)
    res = _lib.residual(store.res_k)
    _lib.call(
        "echokv_write_step", _lib.byref(store.abi), _lib.ptr(store.pages),
        _lib.ptr(key), key.stride(0), key.stride(1), _lib.ptr(value), value.stride(0), value.stride(1),
        _lib.dtype_code(key), _lib.ptr(tok), tok.stride(0), meta.n_rows, _lib.ptr(fin), _lib.ptr(meta.fin_count),
        n_fin, _lib.byref(res), _lib.ptr(kref), ks0, ks1, _lib.stream(),
    )


def finalize_k(store, key: torch.Tensor, meta, full_grid: bool = False) -> None:
    """Quantize each completed K group per channel and store its codes and stats.

    ``full_grid`` launches one program per token row, masked on the device by
    ``meta.fin_count`` (a captured graph does not know the count)."""
    n = meta.n_rows if full_grid else meta.n_fin
    if n == 0 or meta.fin.shape[0] == 0:  # no rows staged: the device count is 0 too
        return
    fin = _fin_rows(store, meta)
    _lib.require_device(key, store.pages)
    key = _kv(key, 0)  # fin rows read only the key rows they name
    # A full grid only reads rows below the device count (<= fin's rows).
    res = _lib.residual(store.res_k)
    _lib.call(
        "echokv_finalize_k", _lib.byref(store.abi), _lib.ptr(store.pages), _lib.ptr(key), key.stride(0),
        key.stride(1), _lib.dtype_code(key), _lib.ptr(fin), _lib.ptr(meta.fin_count), n, _lib.byref(res),
        _lib.stream(),
    )
