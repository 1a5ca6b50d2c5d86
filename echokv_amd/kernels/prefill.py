"""Chunked-prefill attention over a ``TieredKVCache``.

Interface of ``echokv_vllm/kernels/prefill.py`` (``build_tiles`` 56-71,
``build_dequant_work`` 77-87, ``dequant_dense`` 90-115, ``prefill_attention``
170-207). A prefill chunk's queries attend to the request's whole cached
context (this chunk included, already written) with the bottom-right causal
limit: query ``i`` of an ``nq``-token chunk over ``ctx`` keys sees keys
``<= ctx - nq + i``.

One fused HIP kernel (``echokv_amd/csrc/prefill.hip``) serves every chunk
length: each workgroup takes a tile of ``128 // GQA`` query tokens of one
request for one KV head, dequantizes each 32-key tile of the context once
into LDS (fp16) and runs QK^T and PV on MFMA. ``dequant_dense`` keeps the
reference's dense-dequantization entry point (``[total_ctx, H, D]`` K/V).
"""

from __future__ import annotations

import torch

from echokv_amd import _lib
from echokv_amd._util import to_device

ROWS = 128  # query rows (tokens x GQA heads) per workgroup
FUSED_MAX_CHUNK = 1 << 30  # the fused kernel handles every chunk length


def gqa_pad(gqa: int) -> int:
    return 1 << (gqa - 1).bit_length()


def block_m(gqa: int) -> int:
    """Query tokens per tile."""
    return max(1, ROWS // gqa)


def build_tiles(prefill, req_of, gqa: int, device) -> torch.Tensor:
    """Tile table ``[n, 5]`` int32: (q_row0, n_tokens, q_pos0, ctx, request).

    ``prefill`` holds (q_start, q_end, ctx, _) per prefill request, ``req_of``
    the matching block-table row."""
    bm = block_m(gqa)
    rows = []
    for (qs, qe, ctx, *_), r in zip(prefill, req_of):
        nq = qe - qs
        pos0 = ctx - nq
        for t0 in range(0, nq, bm):
            rows.append((qs + t0, min(bm, nq - t0), pos0 + t0, ctx, r))
    tiles = to_device(torch.tensor(rows, dtype=torch.int32).reshape(-1, 5), device)
    return tiles


def build_dequant_work(prefill, req_of, block_size: int, device) -> torch.Tensor:
    """Work list ``[n, 4]`` int32: (request, block index, dense row of block start, ctx);
    entry 4 of each prefill tuple is the context's first dense row."""
    rows = []
    for (_, _, ctx, g0, *_), r in zip(prefill, req_of):
        for bi in range(-(-ctx // block_size)):
            rows.append((r, bi, g0 + bi * block_size, ctx))
    return to_device(torch.tensor(rows, dtype=torch.int32).reshape(-1, 4), device)


def _bt(block_table: torch.Tensor) -> torch.Tensor:
    if block_table.dtype != torch.int32 or block_table.stride(1) != 1:
        block_table = block_table.to(torch.int32).contiguous()
    return block_table


def dequant_dense(store, work: torch.Tensor, total_ctx: int, block_table: torch.Tensor, dtype):
    """Dense ``[total_ctx, H, D]`` K and V (``dtype``) for the contexts in ``work``."""
    L = store.layout
    k = torch.empty(total_ctx, L.num_kv_heads, L.head_size, device=store.device, dtype=dtype)
    v = torch.empty_like(k)
    if work.numel() == 0:
        return k, v
    _lib.require_device(work, block_table, store.pages)
    block_table = _bt(block_table)
    work = work.to(torch.int32).contiguous()
    res = _lib.residual(store.res_k)
    _lib.call(
        "echokv_dequant_dense", _lib.byref(store.abi), _lib.ptr(store.pages), _lib.ptr(store.block_res),
        _lib.ptr(store.res_group), _lib.byref(res), _lib.ptr(work), work.shape[0], _lib.ptr(block_table),
        block_table.stride(0), _lib.ptr(k), _lib.ptr(v), k.stride(0), k.stride(1), _lib.dtype_code(k),
        _lib.stream(),
    )
    return k, v


def prefill_attention(store, query: torch.Tensor, output: torch.Tensor, prefill, req_of, block_table: torch.Tensor,
                      softmax_scale: float, tiles: torch.Tensor | None = None, gather=None, dense=None) -> None:
    """Write attention for every prefill chunk into ``output [T, Hq, D]``.

    ``gather`` / ``dense`` (the reference's alternative inputs) are accepted and
    unused: the fused kernel covers every chunk."""
    if not prefill:
        return
    L = store.layout
    _lib.require_device(query, output, block_table, store.pages)
    hq = query.shape[1]
    gqa = hq // L.num_kv_heads
    if tiles is None:
        tiles = build_tiles(prefill, req_of, gqa, query.device)
    if tiles.numel() == 0:
        return
    if query.stride(2) != 1:
        query = query.contiguous()
    out = output.view(output.shape[0], hq, -1) if output.dim() == 2 else output
    if out.stride(2) != 1:
        raise ValueError("output rows must be contiguous along head_dim")
    block_table = _bt(block_table)
    tiles = tiles.to(torch.int32).contiguous()
    res = _lib.residual(store.res_k)
    _lib.call(
        "echokv_prefill", _lib.byref(store.abi), _lib.ptr(store.pages), _lib.ptr(store.block_res),
        _lib.ptr(store.res_group), _lib.byref(res), _lib.ptr(query), query.stride(0), query.stride(1),
        _lib.dtype_code(query), hq, _lib.ptr(out), out.stride(0), out.stride(1), _lib.dtype_code(out),
        _lib.ptr(tiles), tiles.shape[0], block_m(gqa), _lib.ptr(block_table), block_table.stride(0),
        float(softmax_scale), _lib.stream(),
    )
