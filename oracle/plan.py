"""The per-step write planner, restated group by group in plain Python (oracle;
test infrastructure only).

Restates ``echokv_vllm/write_plan.py:98-240`` (``WritePlanner.plan``): from one
step's slot mapping, which blocks reopen, which K groups finalize (whole in the
step, or completing from the residual), which keys go to which residual slot
(LIFO free list; when none is free, evict the least recently written slot that
no block of the step maps, ties to the slot taken first, and seal its group),
and the K_ref ring rows of the step's last keys. Pinned to the reference's own
plans (``tests/golden/store_*.npz``), then used to check the native planner on
random steps.
"""

from __future__ import annotations

import numpy as np


class PlannerOracle:
    def __init__(self, block_size: int, k_group: int, residual_slots: int, kref_window: int) -> None:
        self.bs, self.kg, self.R, self.W = block_size, k_group, residual_slots, kref_window
        self.stack = [s for s in reversed(range(residual_slots))]  # the last entry is handed out next
        self.owner = {}        # slot -> [block, group, fill, last step, take order]
        self.slot_of = {}      # block -> slot
        self.sealed = {}       # block -> bitmask of sealed groups
        self.step = 0
        self.takes = 0
        self.kref_pos = 0
        self.kref_fill = 0

    def _free(self, slot, res_log):
        b = self.owner.pop(slot)[0]
        self.slot_of.pop(b, None)
        self.stack.append(slot)
        res_log.append((b, -1))

    def plan(self, slot_mapping):
        """Returns (tok [4, n_rows], fin [f, 3 + kg], evictions [e, 4], opened blocks)."""
        self.step += 1
        bs, kg = self.bs, self.kg
        sm = [int(x) for x in slot_mapping]
        n_rows = len(sm)
        tok = np.full((4, n_rows), -1, np.int64)
        tok[0] = sm
        tok[2] = 0
        res_log, evictions = [], []

        writes = [(r, s // bs, s % bs) for r, s in enumerate(sm) if s >= 0]
        opened = sorted({b for _, b, off in writes if off == 0})
        for b in opened:
            if b in self.slot_of:
                self._free(self.slot_of[b], res_log)
            self.sealed.pop(b, None)

        groups = {}  # (block, group) -> [(position, row), ...]
        for r, b, off in writes:
            groups.setdefault((b, off // kg), []).append((off % kg, r))
        keys = sorted(groups)
        for k in keys:
            groups[k].sort(key=lambda pr: pr[0])  # stable: equal positions keep row order

        def is_sealed(b, g):
            return (self.sealed.get(b, 0) >> g) & 1

        whole = {k for k in keys if len(groups[k]) == kg and not is_sealed(*k)}
        done = set()
        for b, g in keys:
            if (b, g) in whole and b not in done:
                done.add(b)
                s = self.slot_of.get(b)
                if s is not None and (b, self.owner[s][1]) in whole:
                    self._free(s, res_log)

        guarded = {self.slot_of[b] for b, _ in keys if b in self.slot_of}
        fin_whole, fin_rest = [], []
        for b, g in keys:
            members = groups[(b, g)]
            if (b, g) in whole:
                fin_whole.append([b, g, -1] + [r for _, r in members])
                continue
            if is_sealed(b, g):
                for _, r in members:
                    tok[2, r] = 1
                continue
            s = self.slot_of.get(b)
            if s is not None and self.owner[s][1] != g:
                s = None
            top = max(p for p, _ in members)
            if top == kg - 1:
                row = [-1] * kg
                for p, r in members:
                    row[p] = r
                fin_rest.append([b, g, -1 if s is None else s] + row)
                if s is not None:
                    self._free(s, res_log)
                continue
            if s is None:
                if not self.stack:
                    cands = [x for x in self.owner if x not in guarded]
                    if not cands:
                        raise RuntimeError("more open K groups than residual slots")
                    v = min(cands, key=lambda x: (self.owner[x][3], self.owner[x][4]))
                    vb, vg, vf = self.owner[v][:3]
                    evictions.append([v, vb, vg, vf])
                    self.sealed[vb] = self.sealed.get(vb, 0) | (1 << vg)
                    self._free(v, res_log)
                s = self.stack.pop()
                self.takes += 1
                self.owner[s] = [b, g, 0, 0, self.takes]
                self.slot_of[b] = s
                guarded.add(s)
                res_log.append((b, s))
            for _, r in members:
                tok[1, r] = s
            self.owner[s][2] = max(self.owner[s][2], top + 1)
            self.owner[s][3] = self.step

        rows = [r for r, _, _ in writes]
        k = min(len(rows), self.W)
        for i, r in enumerate(rows[len(rows) - k :]):
            tok[3, r] = (self.kref_pos + i) % self.W
        self.kref_pos = (self.kref_pos + k) % self.W
        self.kref_fill = min(self.W, self.kref_fill + k)
        fin = np.array(fin_whole + fin_rest, np.int64).reshape(-1, 3 + kg)
        return tok, fin, np.array(evictions, np.int64).reshape(-1, 4), np.array(opened, np.int64), res_log
