"""Paged decode attention over a ``TieredKVCache`` (one query token per sequence).

Interface of ``echokv_vllm/kernels/decode.py:44-92`` (``decode_attention``).
The work runs in two HIP kernels (``echokv_amd/csrc/decode.hip``): a split-KV
MFMA kernel -- one workgroup per (sequence, split), one wave per KV head,
each block's tier read from its page header -- and a log-sum-exp merge that
writes each sequence's output row. Layouts those kernels are not built for
(head sizes other than 64 / 128 up to 256, K groups under 16, block sizes or K
groups that are not powers of two, more than 4 chunks per page) take an fp32
kernel with the same split schedule (``echokv_amd/csrc/decode_any.hip``). A sequence is cut into at most
``num_splits`` splits of ``max(blocks_per_split, ceil(blocks / num_splits))``
blocks, a function of its own length, so its result does not depend on the
rest of the batch.
"""

from __future__ import annotations

import torch

from echokv_amd import _lib

BLOCKS_PER_SPLIT = 16
MAX_SPLITS = 64  # default cap: more, shorter splits keep every CU busy at small batch


def _i64(t: torch.Tensor | None, device) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype != torch.int64 or not t.is_contiguous() or t.device != device:
        t = t.to(device=device, dtype=torch.int64).contiguous()
    return t


def default_splits(block_table: torch.Tensor, block_size: int, blocks_per_split: int, max_len: int | None) -> int:
    max_blocks = block_table.shape[1] if max_len is None else min(block_table.shape[1], -(-max_len // block_size))
    return max(1, min(-(-max_blocks // blocks_per_split), MAX_SPLITS))


def workspace_rows(store, num_q_heads: int, q_dtype: torch.dtype, num_seqs: int, num_splits: int,
                   flags: int) -> int:
    """Rows of ``(acc [rows, Hq, D], ml [rows, Hq, 2])`` a decode call with these arguments uses."""
    rows = _lib.lib().echokv_decode_workspace_rows(_lib.byref(store.abi), num_q_heads, _lib.DTYPES[q_dtype],
                                                   num_seqs, num_splits, flags)
    if rows < 0:
        raise ValueError("decode arguments the kernels do not take")
    return int(rows)


def decode_attention(
    store,
    query: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    softmax_scale: float,
    blocks_per_split: int = BLOCKS_PER_SPLIT,
    q_rows: torch.Tensor | None = None,
    bt_rows: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    max_len: int | None = None,
    num_splits: int | None = None,
    workspace: tuple[torch.Tensor, torch.Tensor] | str | None = None,
    tier: int | None = None,
    batch_invariant: bool = True,
    tier_mask: torch.Tensor | str | None = None,
) -> torch.Tensor:
    """Attention of one query token per sequence over each sequence's cache.

    Sequence ``i`` uses query row ``q_rows[i]`` and block-table row ``bt_rows[i]``
    (default: row ``i``) with cache length ``seq_lens[i]`` (its own token
    included). Without ``out`` returns float32 ``[S, Hq, D]``; with ``out``
    writes sequence ``i`` to ``out[q_rows[i]]`` in ``out``'s dtype; length-0
    sequences (graph padding) leave their row untouched. ``workspace`` =
    caller-owned ``(acc, ml)`` float32 holding ``workspace_rows(...)`` rows of ``Hq * D``
    and ``Hq * 2`` values (``S * splits`` rows at most), or ``"static"``: the
    library's static scratch (no allocation at all, for code under graph capture; at
    most 64 MiB of workspace, and calls on one GPU must not overlap).
    ``tier`` selects the kernel specialised for that tier; by default the tier most
    of the store's blocks are stored at. Blocks of other tiers are read correctly
    either way. With ``batch_invariant`` (the default, as the reference's decode) each
    sequence is split by its own length, so its result does not depend on the rest
    of the batch; ``batch_invariant=False`` spreads the batch's blocks evenly over
    every workgroup the GPU holds instead (faster on uneven batches; a sequence's
    result then depends on the rest of the batch through float rounding).
    ``tier_mask``: for a layer holding blocks at several tiers, each tier's blocks
    on that tier's own fast path (one kernel launch per tier, lowest first, into the
    same partial rows): an int32 device tensor whose element 0 holds the tiers as a
    bit set of tier values (2 | 4 | 8), read when the kernels run, so a captured
    graph follows it from step to step; or ``"auto"``: the tiers the store's pool
    holds blocks at now (one tier: no passes). Needs ``batch_invariant``.
    """
    L = store.layout
    dev = query.device
    _lib.require_device(query, block_table, seq_lens, store.pages)
    s = seq_lens.shape[0]
    hq, d = query.shape[1], query.shape[2]
    if num_splits is None:
        num_splits = default_splits(block_table, L.block_size, blocks_per_split, max_len)
    if query.stride(2) != 1:
        query = query.contiguous()
    if block_table.dtype != torch.int32 or block_table.stride(1) != 1:
        block_table = block_table.to(torch.int32).contiguous()
    lens = _i64(seq_lens, dev)
    q_rows = _i64(q_rows, dev)
    bt_rows = _i64(bt_rows, dev)
    if out is None:
        out = torch.empty(s if q_rows is None else query.shape[0], hq, d, device=dev, dtype=torch.float32)
    if out.stride(2) != 1:
        raise ValueError("out rows must be contiguous along head_dim")
    static = isinstance(workspace, str)
    if static:
        if workspace != "static":
            raise ValueError(f"workspace must be a (acc, ml) pair or 'static', got {workspace!r}")
        acc = ml = None
    else:
        flags = _lib.DECODE_BATCH_INVARIANT if batch_invariant else 0
        rows = workspace_rows(store, hq, query.dtype, s, num_splits, flags)
        if workspace is None:
            acc = torch.empty(rows, hq, d, device=dev, dtype=torch.float32)
            ml = torch.empty(rows, hq, 2, device=dev, dtype=torch.float32)
        else:
            acc, ml = workspace
            if acc.numel() < rows * hq * d or ml.numel() < rows * hq * 2:
                raise ValueError(f"decode workspace holds fewer than the {rows} rows this call needs")
    if isinstance(tier_mask, str):
        if tier_mask != "auto":
            raise ValueError(f"tier_mask must be an int32 device tensor or 'auto', got {tier_mask!r}")
        live = store.pool.live_tiers()
        present = [b for b in (2, 4, 8) if live[b]]
        tier_mask = None
        if len(present) > 1:
            tier_mask = torch.tensor([sum(present)], dtype=torch.int32, device=dev)
    if tier_mask is not None:
        if not batch_invariant:
            raise ValueError("tier passes run on the split schedule: pass batch_invariant=True with tier_mask")
        if tier_mask.dtype != torch.int32 or tier_mask.device != dev or tier_mask.numel() < 1:
            raise ValueError("tier_mask must be an int32 tensor on the query's device")
    if tier is None:
        tier = store.pool.majority_tier()
    res = _lib.residual(store.res_k)
    head = (_lib.byref(store.abi), _lib.ptr(store.pages), _lib.ptr(store.block_res), _lib.ptr(store.res_group),
            _lib.byref(res), _lib.ptr(query), query.stride(0), query.stride(1), _lib.dtype_code(query), hq,
            _lib.ptr(q_rows), _lib.ptr(block_table), block_table.stride(0), _lib.ptr(bt_rows), _lib.ptr(lens), s,
            float(softmax_scale), int(num_splits), int(blocks_per_split), int(tier), _lib.ptr(tier_mask),
            _lib.DECODE_BATCH_INVARIANT if batch_invariant else 0)
    tail = (_lib.ptr(out), out.stride(0), out.stride(1), _lib.dtype_code(out), _lib.stream())
    if static:
        _lib.call("echokv_decode_static", *head, *tail)
    else:
        _lib.call("echokv_decode", *head, _lib.ptr(acc), _lib.ptr(ml), *tail)
    return out
