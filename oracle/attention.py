"""Decode and chunked-prefill attention over dequantized K/V (oracle; tests only).

Restates ``echokv_vllm/kernels/decode.py:95-129`` (one query token per
sequence over its cache, GQA by repeating KV heads) and
``echokv_vllm/kernels/prefill.py:210-236`` (a chunk of ``nq`` queries over a
context of ``ctx`` keys with the bottom-right causal mask: query ``i`` sees
keys ``<= ctx - nq + i``). Softmax and products run in float64.
"""

from __future__ import annotations

import numpy as np


def attend(q, k, v, scale, limit=None):
    """``q [Hq, D]``, ``k, v [n, H, D]`` -> ``[Hq, D]``; keys ``>= limit`` masked."""
    hq, h = q.shape[0], k.shape[1]
    rep = hq // h
    kk = np.repeat(k.astype(np.float64), rep, axis=1)  # [n, Hq, D]
    vv = np.repeat(v.astype(np.float64), rep, axis=1)
    s = np.einsum("hd,nhd->hn", q.astype(np.float64), kk) * scale
    if limit is not None:
        s[:, limit:] = -np.inf
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return np.einsum("hn,nhd->hd", p, vv)


def decode_attention(store, query, block_table, seq_lens, scale, vectorized=False):
    """decode.py:95-129: float ``[S, Hq, D]``. ``vectorized`` reads the cache with the
    store's vectorized gather (same values)."""
    out = np.zeros(query.shape, np.float64)
    for i, n in enumerate(np.asarray(seq_lens).tolist()):
        if vectorized:  # one matrix product per head; a single query sees every key
            pos = np.arange(n)
            k, v = store.gather_vec(np.asarray(block_table[i], np.int64)[pos // store.L.bs], pos % store.L.bs)
            out[i] = attend_causal(query[i][None], k, v, scale)[0]
        else:
            k, v = store.gather_seq(block_table[i], n)
            out[i] = attend(query[i], k, v, scale)
    return out


def prefill_attention(store, query, prefill, req_of, block_table, scale, vectorized=False):
    """prefill.py:210-236: ``prefill`` = [(q_start, q_end, ctx, _)], ``req_of`` = block-table rows.
    ``vectorized`` reads the cache with the vectorized gather and computes each
    (request, query head) as float64 matrix products (same values as the loop)."""
    out = np.zeros(query.shape, np.float64)
    for (qs, qe, ctx, _), r in zip(prefill, req_of):
        nq = qe - qs
        if not vectorized:
            k, v = store.gather_seq(block_table[r], ctx)
            for i in range(nq):
                out[qs + i] = attend(query[qs + i], k, v, scale, limit=ctx - nq + i + 1)
            continue
        pos = np.arange(ctx)
        k, v = store.gather_vec(np.asarray(block_table[r], np.int64)[pos // store.L.bs], pos % store.L.bs)
        out[qs:qe] = attend_causal(query[qs:qe], k, v, scale)
    return out


def prefill_own_group_exact(store, query, key, prefill, req_of, block_table, scale):
    """Prefill with own-group-exact semantics (no counterpart in the reference code:
    ``echokv_vllm`` docs/ECHOKV_VLLM_PLUGIN.md:261-266 describe it as the fix for
    preempted / re-chunked requests): each query attends as decode did when it was
    the newest token. Query ``p`` of a chunk starting at ``c0`` sees the cache
    (``gather``) for keys before its own K group ``[p - p % kg, p]``, and within
    that group the keys as decode saw them while the group was open: full
    precision -- ``key`` rows of this chunk (aligned with the query rows) at
    positions ``>= c0``, the cache before -- with cached V. The group's last
    position is the exception: its write completed the group, which decode then
    read back quantized, so that query sees the cache throughout. Float64."""
    kg = store.L.kg
    out = np.zeros(query.shape, np.float64)
    for (qs, qe, ctx, _), r in zip(prefill, req_of):
        nq = qe - qs
        c0 = ctx - nq
        pos = np.arange(ctx)
        k, v = store.gather_vec(np.asarray(block_table[r], np.int64)[pos // store.L.bs], pos % store.L.bs)
        for g0 in range((c0 // kg) * kg, ctx, kg):  # the own groups of the chunk's queries
            lo, hi = max(g0, c0), min(g0 + kg - 1, ctx)  # open-group queries (and exact keys) in the chunk
            if hi > lo:
                kx = k[:hi].copy()
                kx[lo:hi] = key[qs + lo - c0 : qs + hi - c0]
                out[qs + lo - c0 : qs + hi - c0] = attend_causal(query[qs + lo - c0 : qs + hi - c0], kx, v[:hi],
                                                                 scale)
            last = g0 + kg - 1  # the group's closing query: the cache throughout
            if c0 <= last < ctx:
                out[qs + last - c0] = attend_causal(query[qs + last - c0 : qs + last - c0 + 1], k[: last + 1],
                                                    v[: last + 1], scale)[0]
    return out


def attend_causal(q, k, v, scale):
    """``q [nq, Hq, D]`` over ``k, v [n, H, D]`` with the bottom-right causal limit
    (query i sees keys < n - nq + i + 1), float64, one matrix product per head."""
    nq, hq, _ = q.shape
    n, h = k.shape[0], k.shape[1]
    rep = hq // h
    keep = np.arange(n)[None, :] <= (n - nq + np.arange(nq))[:, None]
    out = np.empty(q.shape, np.float64)
    for hh in range(hq):
        kh = k[:, hh // rep].astype(np.float64)
        s = (q[:, hh].astype(np.float64) @ kh.T) * scale
        s = np.where(keep, s, -np.inf)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, hh] = p @ v[:, hh // rep].astype(np.float64)
    return out
