"""Chunked-prefill attention over a ``TieredKVCache``.

Interface of ``echokv_vllm/kernels/prefill.py`` (``build_tiles`` 56-71,
``build_dequant_work`` 77-87, ``dequant_dense`` 90-115, ``prefill_attention``
170-207). A prefill chunk's queries attend to the request's whole cached
context (this chunk included, already written) with the bottom-right causal
limit: query ``i`` of an ``nq``-token chunk over ``ctx`` keys sees keys
``<= ctx - nq + i``.

Two paths, chosen as the reference chooses (``FUSED_MAX_CHUNK``,
prefill.py:74): when every chunk is at most 64 tokens, one fused HIP kernel
(``echokv_amd/csrc/prefill.hip``): each workgroup takes a tile of
``128 // GQA`` query tokens of one request for one KV head, dequantizes each
32-key tile of the context into LDS (fp16) and runs QK^T and PV on MFMA.
Longer chunks take the two-pass path (``echokv_amd/csrc/prefill_dense.hip``,
the reference's dense dequantization + flash attention, prefill.py:133-167):
every 64-key tile of each context is dequantized once into a workspace, then
a flash-attention kernel with ``256 // GQA``-token query tiles streams it
through LDS. ``dequant_dense`` keeps the reference's dense-dequantization
entry point (``[total_ctx, H, D]`` K/V).

Both kernels are built for head sizes 64 and 128 (and at most ``ROWS`` query
heads per KV head); head size 256 takes the fused kernel at every chunk length,
with half the rows per tile (``rows(256)``: ``64 // GQA`` tokens). Own-group-exact
attention needs head size 64 or 128. Any other layout (the reference's PyTorch
path serves them) takes an fp32 kernel through the same entry point
(``echokv_prefill``): tiles of ``any_block_m(gqa)`` query tokens, so a
workgroup's (token, query head) columns are at most 16, each tile streaming its
causal context once.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from echokv_amd import _lib
from echokv_amd._util import to_device

ROWS = 128  # query rows (tokens x GQA heads) per workgroup of the fused kernel
FUSED_MAX_CHUNK = 64  # the fused kernel only when every chunk is this short
DENSE_ROWS = 256  # query rows per workgroup of the two-pass path
DENSE_KEYS = 64  # keys per workspace tile


def gqa_pad(gqa: int) -> int:
    return 1 << (gqa - 1).bit_length()


def rows(head_size: int = 128) -> int:
    """Query rows (tokens x GQA heads) per workgroup of the fused kernel."""
    return ROWS // 2 if head_size == 256 else ROWS


def block_m(gqa: int, head_size: int = 128) -> int:
    """Query tokens per tile of the fused kernel."""
    return max(1, rows(head_size) // gqa)


def any_block_m(gqa: int) -> int:
    """Query tokens per tile of the fp32 kernel (at most 16 (token, head) columns)."""
    return 1 if gqa >= 16 else 16 // gqa


def build_tiles(prefill, req_of, gqa: int, device, tokens: int | None = None) -> torch.Tensor:
    """Tile table ``[n, 5]`` int32: (q_row0, n_tokens, q_pos0, ctx, request).

    ``prefill`` holds (q_start, q_end, ctx, _) per prefill request, ``req_of``
    the matching block-table row; ``tokens`` per tile, by default ``block_m(gqa)`` (head
    size 64 / 128)."""
    bm = tokens or block_m(gqa)
    rows = []
    for (qs, qe, ctx, *_), r in zip(prefill, req_of):
        nq = qe - qs
        pos0 = ctx - nq
        for t0 in range(0, nq, bm):
            rows.append((qs + t0, min(bm, nq - t0), pos0 + t0, ctx, r))
    tiles = to_device(torch.tensor(rows, dtype=torch.int32).reshape(-1, 5), device)
    tiles.tile_tokens = bm  # checked against the kernel's tile size at launch, without a device read
    return tiles


def check_tiles(tiles: torch.Tensor, tile_m: int) -> None:
    """Refuse a tile table with more query tokens per tile than the kernel takes
    (``tile_m``): the kernel would leave the extra rows unwritten. Tables from
    ``build_tiles`` carry their size; others are read back (a device sync)."""
    if tiles.dim() != 2 or tiles.shape[1] != 5:
        raise ValueError("tiles must be an [n, 5] table (q_row0, n_tokens, q_pos0, ctx, request)")
    made = getattr(tiles, "tile_tokens", None)
    if made is None and tiles.numel():
        made = int(tiles[:, 1].max())
    if made is not None and made > tile_m:
        raise ValueError(f"prefill tiles of {made} query tokens, but this layout's kernel takes at most {tile_m} "
                         "per tile: build them with build_tiles(..., tokens=tile_m)")


class DensePlan(NamedTuple):
    """Device tables of the two-pass path: ``packs [n, 3]`` (block-table row,
    first key, ctx) per 64-key workspace tile and ``qtiles [n, 5]`` (q_row0,
    n_tokens, q_pos0, ctx, first workspace tile of the request's context)."""

    packs: torch.Tensor
    qtiles: torch.Tensor
    tile_m: int


def dense_block_m(gqa: int) -> int:
    """Query tokens per tile of the two-pass path."""
    return max(1, DENSE_ROWS // gqa)


def build_dense_plan(prefill, req_of, gqa: int, device) -> DensePlan:
    """Workspace tiles and query tiles for the two-pass path.

    Query tiles are listed per request, heaviest (most keys) first, requests
    with the most work first, so the longest workgroups start earliest."""
    bm = dense_block_m(gqa)
    packs, groups = [], []
    for (qs, qe, ctx, *_), r in zip(prefill, req_of):
        nq = qe - qs
        t0 = len(packs)
        packs.extend((r, k0, ctx) for k0 in range(0, ctx, DENSE_KEYS))
        pos0 = ctx - nq
        tiles = [(qs + s, min(bm, nq - s), pos0 + s, ctx, t0) for s in range(0, nq, bm)]
        tiles.sort(key=lambda t: -(min(t[3], t[2] + t[1])))
        groups.append((sum(min(t[3], t[2] + t[1]) * t[1] for t in tiles), tiles))
    groups.sort(key=lambda g: -g[0])
    rows = [t for _, tiles in groups for t in tiles]
    packs_t = to_device(torch.tensor(packs, dtype=torch.int32).reshape(-1, 3), device)
    qtiles_t = to_device(torch.tensor(rows, dtype=torch.int32).reshape(-1, 5), device)
    return DensePlan(packs_t, qtiles_t, bm)


def dense_workspace_bytes(store, n_packs: int) -> int:
    n = _lib.lib().echokv_prefill_dense_workspace(_lib.byref(store.abi), n_packs)
    if n < 0:
        raise RuntimeError(f"echokv_prefill_dense_workspace: {_lib.lib().echokv_error_string(int(-n)).decode()}")
    return int(n)


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


def _out_view(output: torch.Tensor, hq: int) -> torch.Tensor:
    out = output.view(output.shape[0], hq, -1) if output.dim() == 2 else output
    if out.stride(2) != 1:
        raise ValueError("output rows must be contiguous along head_dim")
    return out


def kernels_take(head_size: int, gqa: int) -> bool:
    """Whether the MFMA prefill kernels serve this layout (else the fp32 kernel)."""
    return head_size in (64, 128, 256) and gqa <= rows(head_size)


def own_group_takes(head_size: int, gqa: int) -> bool:
    """Whether own-group-exact prefill serves this layout (head size 64 or 128)."""
    return head_size in (64, 128) and kernels_take(head_size, gqa)


def use_dense(prefill, head_size: int) -> bool:
    """The two-pass path serves a batch with any chunk longer than FUSED_MAX_CHUNK."""
    return head_size in (64, 128) and any(qe - qs > FUSED_MAX_CHUNK for qs, qe, *_ in prefill)


def prefill_attention_dense(store, query: torch.Tensor, output: torch.Tensor, prefill, req_of,
                            block_table: torch.Tensor, softmax_scale: float, plan: DensePlan | None = None,
                            workspace: torch.Tensor | None = None, lse: torch.Tensor | None = None) -> None:
    """Two-pass prefill (echokv_vllm/kernels/prefill.py:133-167): dequantize each
    context once into a workspace of 64-key tiles, then flash attention over it.
    ``plan`` / ``workspace`` (uint8, ``dense_workspace_bytes``) may be built once per
    step and shared by every layer. With ``lse`` (float32 ``[T, Hq]``) each query's
    own K group is left out and the rows' log-sum-exp written (own-group-exact part 1)."""
    if not prefill:
        return
    L = store.layout
    _lib.require_device(query, output, block_table, store.pages)
    hq = query.shape[1]
    gqa = hq // L.num_kv_heads
    if plan is None:
        plan = build_dense_plan(prefill, req_of, gqa, query.device)
    n_q = plan.qtiles.shape[0]
    if n_q == 0:
        return
    if query.stride(2) != 1:
        query = query.contiguous()
    out = _out_view(output, hq)
    block_table = _bt(block_table)
    n_packs = plan.packs.shape[0]
    ws_bytes = dense_workspace_bytes(store, n_packs)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=query.device)
    elif workspace.dtype != torch.uint8 or workspace.numel() < ws_bytes:
        raise ValueError(f"prefill workspace holds {workspace.numel()} bytes, the plan needs {ws_bytes}")
    ws = workspace
    res = _lib.residual(store.res_k)
    _lib.call(
        "echokv_prefill_dense", _lib.byref(store.abi), _lib.ptr(store.pages), _lib.ptr(store.block_res),
        _lib.ptr(store.res_group), _lib.byref(res), _lib.ptr(query), query.stride(0), query.stride(1),
        _lib.dtype_code(query), hq, _lib.ptr(out), out.stride(0), out.stride(1), _lib.dtype_code(out),
        _lib.ptr(plan.packs), n_packs, _lib.ptr(plan.qtiles), n_q, plan.tile_m, _lib.ptr(block_table),
        block_table.stride(0), _lib.ptr(ws), ws_bytes, float(softmax_scale), int(lse is not None), _lib.ptr(lse),
        _lib.stream(),
    )


def prefill_attention(store, query: torch.Tensor, output: torch.Tensor, prefill, req_of, block_table: torch.Tensor,
                      softmax_scale: float, tiles: torch.Tensor | None = None, gather=None, dense=None,
                      own_group_key: torch.Tensor | None = None, own_group_rows: torch.Tensor | None = None) -> None:
    """Write attention for every prefill chunk into ``output [T, Hq, D]``.

    A batch with a chunk longer than ``FUSED_MAX_CHUNK`` takes the two-pass
    path; ``dense`` carries its step-wide inputs, built once for every layer: a
    ``DensePlan`` or ``(DensePlan, workspace)`` (the reference builder's dense
    tuple has the same role). Otherwise the fused kernel over ``tiles``.
    ``gather`` (the reference's PyTorch-path index) is accepted and unused.

    ``own_group_key`` (this step's key rows ``[T, H, D]``, aligned with the query
    rows) turns on own-group-exact attention: each query sees its own K group at
    full precision, as decode saw it while the group was open (the chunk's keys
    from ``own_group_key``, earlier ones of the group from the cache); the rest of
    the context as usual. ``own_group_rows`` (``own_group_rows(prefill, req_of)``)
    may be built once per step."""
    if not prefill:
        return
    gqa = query.shape[1] // store.layout.num_kv_heads
    if own_group_key is not None and not own_group_takes(store.layout.head_size, gqa):
        raise ValueError("own-group-exact prefill needs head size 64 or 128 and at most 128 query heads per KV head")
    if not kernels_take(store.layout.head_size, gqa):
        prefill_attention_fused(store, query, output, prefill, req_of, block_table, softmax_scale)
        return
    part, lse = output, None
    if own_group_key is not None:
        n = query.shape[0]
        part = torch.empty(n, query.shape[1], store.layout.head_size, device=query.device, dtype=torch.float32)
        lse = torch.empty(n, query.shape[1], device=query.device, dtype=torch.float32)
    if use_dense(prefill, store.layout.head_size):
        plan, ws = (dense, None) if isinstance(dense, DensePlan) else (dense or (None, None))
        if plan is not None and not isinstance(plan, DensePlan):
            raise ValueError("dense must be a DensePlan or a (DensePlan, workspace) pair")
        prefill_attention_dense(store, query, part, prefill, req_of, block_table, softmax_scale, plan, ws, lse)
    else:
        prefill_attention_fused(store, query, part, prefill, req_of, block_table, softmax_scale, tiles, lse)
    if own_group_key is not None:
        rows = own_group_rows if own_group_rows is not None else build_own_group_rows(prefill, req_of, query.device)
        own_group_merge(store, query, own_group_key, rows, block_table, part, lse, output, softmax_scale)


def build_own_group_rows(prefill, req_of, device) -> torch.Tensor:
    """Rows ``[T, 4]`` int32 of the own-group part: (query row, position, the chunk's
    first position, block-table row) per query token."""
    parts = []
    for (qs, qe, ctx, *_), r in zip(prefill, req_of):
        nq = qe - qs
        c0 = ctx - nq
        i = torch.arange(nq, dtype=torch.int32)
        parts.append(torch.stack([qs + i, c0 + i, torch.full_like(i, c0), torch.full_like(i, r)], 1))
    rows = torch.cat(parts) if parts else torch.zeros(0, 4, dtype=torch.int32)
    return to_device(rows.contiguous(), device)


def own_group_merge(store, query: torch.Tensor, key: torch.Tensor, rows: torch.Tensor, block_table: torch.Tensor,
                    part: torch.Tensor, lse: torch.Tensor, output: torch.Tensor, softmax_scale: float) -> None:
    """Own-group-exact part 2 (``echokv_prefill_own_group``): each row's own K group
    with full-precision keys, merged with ``part`` / ``lse`` into ``output``."""
    if rows.shape[0] == 0:
        return
    L = store.layout
    _lib.require_device(query, key, rows, block_table, part, lse, output, store.pages)
    hq = query.shape[1]
    if query.stride(2) != 1:
        query = query.contiguous()
    if key.stride(2) != 1:
        key = key.contiguous()
    if part.dtype != torch.float32 or part.stride(2) != 1 or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("part must be float32 rows, lse float32 [T, Hq] contiguous")
    out = _out_view(output, hq)
    rows = rows.to(torch.int32).contiguous()
    block_table = _bt(block_table)
    res = _lib.residual(store.res_k)
    _lib.call(
        "echokv_prefill_own_group", _lib.byref(store.abi), _lib.ptr(store.pages), _lib.ptr(store.block_res),
        _lib.ptr(store.res_group), _lib.byref(res), _lib.ptr(query), query.stride(0), query.stride(1),
        _lib.dtype_code(query), hq, _lib.ptr(key), key.stride(0), key.stride(1), _lib.dtype_code(key),
        _lib.ptr(rows), rows.shape[0], _lib.ptr(block_table), block_table.stride(0), _lib.ptr(part), part.stride(0),
        part.stride(1), _lib.ptr(lse), _lib.ptr(out), out.stride(0), out.stride(1), _lib.dtype_code(out),
        float(softmax_scale), _lib.stream(),
    )


def prefill_attention_fused(store, query: torch.Tensor, output: torch.Tensor, prefill, req_of,
                            block_table: torch.Tensor, softmax_scale: float, tiles: torch.Tensor | None = None,
                            lse: torch.Tensor | None = None) -> None:
    """The fused kernel (echokv_vllm/kernels/prefill.py:242-327) over ``tiles``; ``lse`` as
    for ``prefill_attention_dense``. Layouts the MFMA kernel is not built for take the
    fp32 kernel (tiles of ``any_block_m(gqa)`` tokens)."""
    if not prefill:
        return
    L = store.layout
    hq = query.shape[1]
    gqa = hq // L.num_kv_heads
    tile_m = block_m(gqa, L.head_size) if kernels_take(L.head_size, gqa) else any_block_m(gqa)
    if tiles is not None:
        check_tiles(tiles, tile_m)
    _lib.require_device(query, output, block_table, store.pages)
    if tiles is None:
        tiles = build_tiles(prefill, req_of, gqa, query.device, tokens=tile_m)
    if tiles.numel() == 0:
        return
    if query.stride(2) != 1:
        query = query.contiguous()
    out = _out_view(output, hq)
    block_table = _bt(block_table)
    tiles = tiles.to(torch.int32).contiguous()
    res = _lib.residual(store.res_k)
    _lib.call(
        "echokv_prefill", _lib.byref(store.abi), _lib.ptr(store.pages), _lib.ptr(store.block_res),
        _lib.ptr(store.res_group), _lib.byref(res), _lib.ptr(query), query.stride(0), query.stride(1),
        _lib.dtype_code(query), hq, _lib.ptr(out), out.stride(0), out.stride(1), _lib.dtype_code(out),
        _lib.ptr(tiles), tiles.shape[0], tile_m, _lib.ptr(block_table), block_table.stride(0),
        float(softmax_scale), int(lse is not None), _lib.ptr(lse), _lib.stream(),
    )
