"""Host planning of one engine step's KV writes, shared by every layer.

Interface of ``echokv_vllm/write_plan.py`` (``Eviction`` 28-33, ``WritePlan``
40-74, ``WritePlanner`` 77-240, ``SharedState`` 243-271, ``WriteMeta`` 274-282,
``stage_plan`` 285-315). The planning runs in native code
(``echokv_amd/host/plan.cpp`` through ``libechokv_host.so``): from the step's slot
mapping it decides, without looking at tensor values,

* which blocks (re)open (a write at offset 0);
* which K groups complete (one ``fin`` row each: the token row of every position,
  or -1 where the key already sits in the residual);
* which keys of still-open groups go to a residual slot, evicting (sealing) the
  least recently written unprotected slot when none is free;
* where the step's last ``kref_window`` keys land in the K_ref ring;

and writes the result as the int64 image the device reads, so staging a plan is
one pinned host-to-device copy. This module wraps the native objects with the
reference's classes and attribute names.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from echokv_amd import _host
from echokv_amd._util import to_device


@dataclass
class Eviction:
    """A residual slot evicted this step: its group is sealed with ``fill`` tokens."""

    slot: int
    block: int
    group: int
    fill: int


def _none() -> np.ndarray:
    return np.zeros(0, dtype=np.int64)


@dataclass
class WritePlan:
    """One step's writes as host arrays (views into ``stage``, the device image).

    Per token row: ``tok_slot`` (-1 = no write), ``tok_res`` (residual slot or
    -1), ``tok_sealed`` (1 = quantize the key under the group's stored stats),
    ``tok_kref`` (K_ref row or -1). ``fin [f, 3 + k_group]``: ``[block, group,
    residual slot or -1, token row per position (-1 = residual)]``.
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
    stage: np.ndarray = field(default_factory=_none)  # [n_fin | tok | fin | residual map | residual groups]
    touched: np.ndarray = field(default_factory=lambda: np.zeros((0, 3), np.int64))

    @property
    def n_fin(self) -> int:
        return int(self.fin.shape[0])


class WritePlanner:
    """Residual-slot allocator and K_ref cursor of one KV cache group.

    ``num_blocks`` fixes the per-block arrays (as ``SharedState`` does); without it
    they grow with the slots seen, as a standalone planner needs."""

    def __init__(self, block_size: int, k_group: int, residual_slots: int, kref_window: int = 64,
                 num_blocks: int | None = None) -> None:
        lib = _host.lib()
        h = lib.ekh_planner_new(num_blocks or 0, block_size, k_group, residual_slots, kref_window)
        if not h:
            raise ValueError(f"bad planner shape: block_size {block_size}, k_group {k_group}, "
                             f"residual_slots {residual_slots}, kref_window {kref_window}")
        self._h = C.c_void_p(h)
        self._free_fn = lib.ekh_planner_free
        self.bs = block_size
        self.g = k_group
        self.num_slots = residual_slots
        self.kref_window = kref_window

    def __del__(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._free_fn(h)
            self._h = None

    def _state(self, what: int) -> int:
        return int(_host.lib().ekh_planner_state(self._h, what))

    @property
    def step(self) -> int:
        return self._state(_host.STEP)

    @property
    def kref_pos(self) -> int:
        return self._state(_host.KREF_POS)

    @property
    def kref_fill(self) -> int:
        return self._state(_host.KREF_FILL)

    @property
    def free(self) -> list:
        """The free residual slots, bottom to top (the last is handed out next)."""
        out = np.zeros(self.num_slots, np.int64)
        n = _host.lib().ekh_residual_free_list(self._h, _host.i64p(out), out.size)
        return out[:n].tolist()

    def sealed_mask(self, block: int) -> int:
        return int(_host.lib().ekh_sealed_mask(self._h, int(block)))

    @property
    def sealed(self) -> dict:
        """block -> bitmask of its K groups sealed by an eviction (nonzero entries)."""
        n = self._state(_host.NUM_BLOCKS)
        return {b: m for b in range(n) if (m := self.sealed_mask(b))}

    def plan(self, slot_mapping_cpu) -> WritePlan:
        sm = slot_mapping_cpu.numpy() if torch.is_tensor(slot_mapping_cpu) else slot_mapping_cpu
        sm = _host.as_i64(sm)
        v = _host.PlanView()
        rc = _host.lib().ekh_plan(self._h, _host.i64p(sm), sm.size, C.byref(v))
        if rc == _host.ESLOTS:
            raise RuntimeError(f"more than {self.num_slots} open K groups in one step")
        if rc != _host.OK:
            raise ValueError("slot mapping names a block past the planner's pool")
        return _plan_from_view(v, self.bs, self.g)


def _plan_from_view(v: _host.PlanView, bs: int, g: int) -> WritePlan:
    stage = _host.copy_i64(v.stage, v.stage_len)
    t, f, w = v.n_rows, v.n_fin, 3 + g
    o = 1 + 4 * t
    tok = stage[1:o].reshape(4, t)
    fin = stage[o : o + f * w].reshape(f, w)
    o += f * w
    maps = []
    for n in (v.n_res_map, v.n_res_map, v.n_grp_map, v.n_grp_map):
        maps.append(stage[o : o + n])
        o += n
    ev = _host.copy_i64(v.evict, 4 * v.n_evict).reshape(-1, 4)
    touched = _host.copy_i64(v.touched, 3 * v.n_touched).reshape(-1, 3)
    return WritePlan(
        step=int(v.step), n_rows=int(t), tok_slot=tok[0], tok_res=tok[1], tok_sealed=tok[2], tok_kref=tok[3],
        fin=fin, evictions=[Eviction(*map(int, e)) for e in ev], open_np=_host.copy_i64(v.open, v.n_open),
        touched_np=touched[:, 0], touched_fill=touched[:, 1], touched_count=touched[:, 2],
        res_map_block=maps[0], res_map_value=maps[1], res_group_slot=maps[2], res_group_value=maps[3],
        block_size=bs, k_group=g, stage=stage, touched=touched)


class SharedState:
    """What every layer of one KV cache group shares (``write_plan.py:243-271``):
    the planner, per-block host bookkeeping (``fill_h``, ``last_h``, ``cum_h``:
    numpy views of the native arrays) and the device residual map read by the
    attention kernels."""

    def __init__(self, num_blocks: int, block_size: int, k_group: int, residual_slots: int,
                 kref_window: int, device) -> None:
        self.num_blocks = num_blocks
        self.planner = WritePlanner(block_size, k_group, residual_slots, kref_window, num_blocks=num_blocks)
        lib = _host.lib()
        self.fill_h, self.last_h, self.cum_h = (
            _host.view_i64(lib.ekh_block_array(self.planner._h, which), num_blocks, self.planner)
            for which in (_host.FILL, _host.LAST, _host.CUM))
        self.block_res = torch.full((num_blocks,), -1, dtype=torch.long, device=device)
        self.res_group = torch.zeros(residual_slots + 1, dtype=torch.long, device=device)

    def commit(self, plan: WritePlan) -> None:
        """Record the step's touched blocks (after every layer prepared the step)."""
        t = np.ascontiguousarray(plan.touched)
        rc = _host.lib().ekh_commit(self.planner._h, plan.step, _host.i64p(t), t.shape[0])
        if rc != _host.OK:
            raise ValueError("plan names a block past this cache group's pool")

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
    """``plan.stage`` (and ``opened`` = (block ids, headers ``[rows, 16]`` uint8) -- one
    layer's rows, or several layers' one after another) in one host-to-device copy:
    returns ``(WriteMeta, (res blocks, res values, group slots, group values, opened
    ids, headers))``."""
    t, f, w = plan.n_rows, plan.n_fin, 3 + plan.k_group
    image = plan.stage
    n_open = n_hdr = 0
    if opened is not None:
        ids = _host.as_i64(opened[0])
        n_open = ids.size
        hdr = np.ascontiguousarray(opened[1]).view(np.int64).reshape(-1)
        n_hdr = hdr.size
        image = np.concatenate([image, ids, hdr])
    dev = to_device(torch.from_numpy(image), device)
    o = 1 + 4 * t
    meta = WriteMeta(tok=dev[1:o].view(4, t), fin=dev[o : o + f * w].view(f, w), fin_count=dev[0:1], n_rows=t,
                     n_fin=f)
    o += f * w
    maps = []
    for n in (plan.res_map_block.size, plan.res_map_value.size, plan.res_group_slot.size, plan.res_group_value.size):
        maps.append(dev[o : o + n])
        o += n
    headers = (None, None)
    if opened is not None:
        headers = (dev[o : o + n_open], dev[o + n_open : o + n_open + n_hdr].view(-1, 2).view(torch.uint8))
    return meta, (*maps, *headers)
