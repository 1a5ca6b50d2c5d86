"""Host planning of one engine step's KV writes, shared by every layer.

Interface of ``echokv_vllm/write_plan.py`` (``Eviction`` 28-33, ``WritePlan``
40-74, ``WritePlanner.plan`` 98-240, ``SharedState`` 243-271, ``WriteMeta``
274-282, ``stage_plan`` 285-315). Everything a write decides without looking
at tensor values is computed here from the slot mapping, once per step, as
numpy arrays indexed by token row:

* blocks (re)opened this step (a write at offset 0);
* K groups that complete this step (one ``fin`` row each, naming the token
  row of every position, or -1 where the key is already in the residual);
* keys of still-open groups, which go to a residual slot; a slot is taken
  from a LIFO free list, and when none is free the least recently written
  unprotected slot is evicted (its group is *sealed*: quantized with the
  tokens present, later tokens reuse those stats);
* the K_ref ring row of the step's last ``kref_window`` keys.

The device only ever sees ``WriteMeta`` (the write kernels' input contract)
and index updates, so a captured HIP graph replays the step unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from echokv_amd._util import to_device


@dataclass
class Eviction:
    slot: int
    block: int
    group: int
    fill: int


def _none() -> np.ndarray:
    return np.zeros(0, dtype=np.int64)


@dataclass
class WritePlan:
    """One step's writes as host arrays (``write_plan.py:40-74``).

    Per token row: ``tok_slot`` (-1 = no write), ``tok_res`` (residual slot
    or -1), ``tok_sealed`` (1 = quantize the key under the group's stored
    stats), ``tok_kref`` (K_ref row or -1). ``fin [f, 3 + k_group]``:
    ``[block, group, residual slot or -1, token row per position (-1 = residual)]``.
    """

    step: int
    n_rows: int
    tok_slot: np.ndarray
    tok_res: np.ndarray
    tok_sealed: np.ndarray
    tok_kref: np.ndarray
    fin: np.ndarray
    evictions: list = field(default_factory=list)
    open_np: np.ndarray = field(default_factory=_none)
    touched_np: np.ndarray = field(default_factory=_none)
    touched_fill: np.ndarray = field(default_factory=_none)
    touched_count: np.ndarray = field(default_factory=_none)
    res_map_block: np.ndarray = field(default_factory=_none)
    res_map_value: np.ndarray = field(default_factory=_none)
    res_group_slot: np.ndarray = field(default_factory=_none)
    res_group_value: np.ndarray = field(default_factory=_none)
    block_size: int = 0
    k_group: int = 0

    @property
    def n_fin(self) -> int:
        return int(self.fin.shape[0])


class WritePlanner:
    """Residual-slot allocator and K_ref cursor of one KV cache group."""

    def __init__(self, block_size: int, k_group: int, residual_slots: int, kref_window: int = 64) -> None:
        self.bs = block_size
        self.g = k_group
        self.num_slots = residual_slots
        # LIFO free list: slot 0 is handed out first, a released slot next.
        self.free: list[int] = list(range(residual_slots - 1, -1, -1))
        self.block_slot: dict[int, int] = {}
        # slot -> [block, group, fill, last step]; insertion order breaks
        # recency ties when choosing an eviction victim.
        self.slot_info: dict[int, list[int]] = {}
        self.sealed: dict[int, int] = {}  # block -> bitmask of sealed groups
        self.step = 0
        self.kref_window = kref_window
        self.kref_pos = 0
        self.kref_fill = 0

    def _release(self, slot: int, res_ops: list) -> None:
        blk = self.slot_info.pop(slot)[0]
        self.block_slot.pop(blk, None)
        self.free.append(slot)
        res_ops.append((blk, -1))

    def _take_slot(self, blk: int, grp: int, protected: set, res_ops: list, grp_ops: list,
                   evictions: list) -> int:
        if not self.free:
            victims = [s for s in self.slot_info if s not in protected]
            if not victims:
                raise RuntimeError(f"more than {self.num_slots} open K groups in one step")
            v = min(victims, key=lambda s: self.slot_info[s][3])
            vb, vg, vf, _ = self.slot_info[v]
            evictions.append(Eviction(v, vb, vg, vf))
            self.sealed[vb] = self.sealed.get(vb, 0) | (1 << vg)
            self._release(v, res_ops)
        s = self.free.pop()
        self.slot_info[s] = [blk, grp, 0, 0]
        self.block_slot[blk] = s
        protected.add(s)
        res_ops.append((blk, s))
        grp_ops.append((s, grp))
        return s

    def plan(self, slot_mapping_cpu) -> WritePlan:
        self.step += 1
        bs, g = self.bs, self.g
        sm = np.asarray(slot_mapping_cpu.numpy() if torch.is_tensor(slot_mapping_cpu) else slot_mapping_cpu)
        sm = sm.astype(np.int64).reshape(-1)
        n_rows = sm.size
        rows = np.flatnonzero(sm >= 0)
        slots = sm[rows]
        n = slots.size
        blk = slots // bs
        off = slots % bs
        grp = off // g
        pos = off % g

        res_ops: list = []  # (block, slot or -1) in order; the last one per block wins
        grp_ops: list = []  # (slot, group)
        opened = np.unique(blk[off == 0])
        for b in opened.tolist():
            s = self.block_slot.get(b)
            if s is not None:
                self._release(s, res_ops)
            self.sealed.pop(b, None)

        # Tokens grouped by (block, K group), positions ascending inside each.
        gkey = blk * (bs // g) + grp
        order = np.lexsort((pos, gkey))
        if n:
            sk = gkey[order]
            starts = np.flatnonzero(np.r_[True, sk[1:] != sk[:-1]])
        else:
            starts = _none()
        counts = np.diff(np.r_[starts, n]).astype(np.int64)
        first = order[starts]
        ublk, ugrp = blk[first], grp[first]

        # Whole groups inside this batch (prefill): finalize straight from the
        # key rows, no residual involved.
        whole = counts == g
        if self.sealed:
            whole &= np.array([not ((self.sealed.get(int(b), 0) >> int(r)) & 1) for b, r in zip(ublk, ugrp)],
                              dtype=bool)
        wi = np.flatnonzero(whole)
        if wi.size:
            whole_rows = rows[order[starts[wi][:, None] + np.arange(g)]]
        else:
            whole_rows = np.zeros((0, g), np.int64)
        for b in ublk[wi].tolist():  # a group rewritten while its slot was open (rare)
            s = self.block_slot.get(b)
            if s is not None and self.slot_info[s][1] in set(ugrp[wi][ublk[wi] == b].tolist()):
                self._release(s, res_ops)

        tok_res = np.full(n, -1, np.int64)
        tok_sealed = np.zeros(n, np.int64)
        fin_head, fin_rows, evictions = [], [], []
        protected = {self.block_slot[b] for b in np.unique(blk).tolist() if b in self.block_slot}
        for u in np.flatnonzero(~whole).tolist():
            idx = order[starts[u] : starts[u] + counts[u]]
            b, r = int(ublk[u]), int(ugrp[u])
            p = pos[idx]
            if (self.sealed.get(b, 0) >> r) & 1:
                tok_sealed[idx] = 1
                continue
            s = self.block_slot.get(b)
            if s is not None and self.slot_info[s][1] != r:
                s = None
            top = int(p.max())
            if top == g - 1:  # the group completes now
                fin_head.append((b, r, -1 if s is None else s))
                rr = np.full(g, -1, np.int64)
                rr[p] = rows[idx]
                fin_rows.append(rr)
                if s is not None:
                    self._release(s, res_ops)
                continue
            if s is None:
                s = self._take_slot(b, r, protected, res_ops, grp_ops, evictions)
            tok_res[idx] = s
            info = self.slot_info[s]
            info[2] = max(info[2], top + 1)
            info[3] = self.step

        head = np.concatenate([
            np.stack([ublk[wi], ugrp[wi], np.full(wi.size, -1, np.int64)], 1).reshape(-1, 3),
            np.asarray(fin_head, np.int64).reshape(-1, 3),
        ])
        body = np.concatenate([whole_rows.reshape(-1, g), np.asarray(fin_rows, np.int64).reshape(-1, g)])
        fin = np.concatenate([head, body], 1).astype(np.int64)

        # Per touched block: highest offset written + 1, and token count.
        if n:
            bsorted = blk[order]
            bstarts = np.flatnonzero(np.r_[True, bsorted[1:] != bsorted[:-1]])
            touched = bsorted[bstarts]
            touched_fill = np.maximum.reduceat(off[order] + 1, bstarts)
            touched_count = np.diff(np.r_[bstarts, n]).astype(np.int64)
        else:
            touched = touched_fill = touched_count = _none()

        # The step's last kref_window keys enter the K_ref ring in order.
        k = min(n, self.kref_window)
        kref = np.full(n, -1, np.int64)
        if k:
            kref[n - k :] = (self.kref_pos + np.arange(k)) % self.kref_window
            self.kref_pos = (self.kref_pos + k) % self.kref_window
            self.kref_fill = min(self.kref_window, self.kref_fill + k)

        def per_row(a):
            o = np.full(n_rows, -1, np.int64)
            o[rows] = a
            return o

        res_map = dict(res_ops)
        grp_map = dict(grp_ops)
        return WritePlan(
            step=self.step, n_rows=n_rows, tok_slot=sm, tok_res=per_row(tok_res),
            tok_sealed=np.maximum(per_row(tok_sealed), 0), tok_kref=per_row(kref), fin=fin,
            evictions=evictions, open_np=opened, touched_np=touched, touched_fill=touched_fill,
            touched_count=touched_count,
            res_map_block=np.fromiter(res_map.keys(), np.int64, len(res_map)),
            res_map_value=np.fromiter(res_map.values(), np.int64, len(res_map)),
            res_group_slot=np.fromiter(grp_map.keys(), np.int64, len(grp_map)),
            res_group_value=np.fromiter(grp_map.values(), np.int64, len(grp_map)),
            block_size=bs, k_group=g,
        )


class SharedState:
    """State every layer of one KV cache group shares (``write_plan.py:243-271``):
    the planner, per-block host bookkeeping, and the device residual map read
    by the attention kernels."""

    def __init__(self, num_blocks: int, block_size: int, k_group: int, residual_slots: int,
                 kref_window: int, device) -> None:
        self.num_blocks = num_blocks
        self.planner = WritePlanner(block_size, k_group, residual_slots, kref_window)
        self.fill_h = np.zeros(num_blocks, np.int64)
        self.last_h = np.zeros(num_blocks, np.int64)
        self.cum_h = np.zeros(num_blocks, np.int64)
        self.block_res = torch.full((num_blocks,), -1, dtype=torch.long, device=device)
        self.res_group = torch.zeros(residual_slots + 1, dtype=torch.long, device=device)

    def commit(self, plan: WritePlan) -> None:
        t = plan.touched_np
        if t.size:
            self.fill_h[t] = np.maximum(self.fill_h[t], plan.touched_fill)
            self.last_h[t] = plan.step
            self.cum_h[t] += plan.touched_count

    def apply_res_map(self, blocks, values, slots, groups) -> None:
        if blocks.numel():
            self.block_res[blocks] = values
        if slots.numel():
            self.res_group[slots] = groups


@dataclass
class WriteMeta:
    """The write kernels' device inputs (``write_plan.py:274-282``)."""

    tok: torch.Tensor  # [4, >= n_rows] int64: slot, residual slot, sealed, K_ref row
    fin: torch.Tensor  # [>= n_fin, 3 + k_group] int64
    fin_count: torch.Tensor  # [1] int64: masks a full-grid (graph) finalize
    n_rows: int
    n_fin: int


def stage_plan(plan: WritePlan, device, opened=None):
    """One host-to-device copy of ``plan`` (and of ``opened`` headers): ``(WriteMeta, extra)``
    with ``extra = (res blocks, res values, group slots, group values, opened ids, headers)``."""
    t, f, w = plan.n_rows, plan.n_fin, 3 + plan.k_group
    parts = [np.array([f]), plan.tok_slot, plan.tok_res, plan.tok_sealed, plan.tok_kref, plan.fin,
             plan.res_map_block, plan.res_map_value, plan.res_group_slot, plan.res_group_value]
    if opened is not None:
        parts += [opened[0], np.ascontiguousarray(opened[1]).view(np.int64)]
    flat = [np.asarray(p, dtype=np.int64).reshape(-1) for p in parts]
    dev = to_device(torch.from_numpy(np.concatenate(flat)), device)
    views, o = [], 0
    for a in flat:
        views.append(dev[o : o + a.size])
        o += a.size
    meta = WriteMeta(tok=dev[1 : 1 + 4 * t].view(4, t), fin=views[5].view(f, w), fin_count=views[0],
                     n_rows=t, n_fin=f)
    headers = (None, None)
    if opened is not None:
        headers = (views[10], views[11].view(-1, 2).view(torch.uint8))
    return meta, (*views[6:10], *headers)
