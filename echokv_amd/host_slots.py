"""Slot mapping and sequence lengths on the host, without waiting for the GPU.

Interface of ``echokv_vllm/host_slots.py:115-195`` (``install``, ``install_v2``,
``install_v1_dummy``, ``is_dummy_step``, ``host_lens_and_slots``). vLLM computes
``slot_mapping`` on the device; copying it back would wait for the stream to
drain and stop the host from preparing step N+1 while the GPU runs step N. The
write planner needs it on the host, so this module derives it from host-side
copies:

* positions from ``query_start_loc_cpu`` and ``seq_lens_cpu_upper_bound``;
* block ids from a host copy of the block table: the V1 runner's
  ``BlockTable.block_table.np`` (indexed by batch row), or, for the V2 runner's
  ``BlockTables`` (device tables indexed by request slot), a numpy mirror of every
  ``append_block_ids`` write plus ``cm.req_idx`` (batch row -> slot).

Dummy steps (warm-up, profiling, graph capture, idle data-parallel ranks) write
nothing -- their device slot mapping is all -1 -- while their block-table rows
may belong to live requests, so they are recognised and left to the device copy.
The hooks are installed by patching the vLLM classes once (idempotent).
"""

from __future__ import annotations

import functools
import weakref

import numpy as np
import torch

_MARK = "_echokv_hook"


class _Registry:
    """Every live V1 / V2 block table, and whether a V1 dummy run is on the stack."""

    def __init__(self) -> None:
        self.v1 = weakref.WeakSet()
        self.v2 = weakref.WeakSet()
        self.v1_dummy_depth = 0

    def v1_match(self, ptr: int):
        for t in list(self.v1):
            bt = getattr(t, "block_table", None)
            if bt is not None and bt.gpu.data_ptr() == ptr:
                return t
        return None

    def v2_match(self, ptr: int):
        for t in list(self.v2):
            for i, inp in enumerate(t.input_block_tables):
                if inp.data_ptr() == ptr:
                    return t, i
        return None


REG = _Registry()


def _patch(cls, name: str, wrap) -> None:
    """Replace ``cls.name`` with ``wrap(original)`` unless it is already hooked."""
    orig = getattr(cls, name)
    if getattr(orig, _MARK, False):
        return
    new = functools.wraps(orig)(wrap(orig))
    setattr(new, _MARK, True)
    setattr(cls, name, new)


def _track_instances(cls, registry: weakref.WeakSet, on_init=None) -> None:
    def wrap(orig):
        def __init__(self, *args, **kwargs):
            orig(self, *args, **kwargs)
            if on_init is not None:
                on_init(self)
            registry.add(self)
        return __init__
    _patch(cls, "__init__", wrap)


def _mirror_tables(tables) -> None:
    """A host copy of each of a V2 ``BlockTables``' device tables."""
    tables._echokv_host = [np.zeros(tuple(b.gpu.shape), np.int64) for b in tables.block_tables]


def install_v2(cls) -> None:
    """Mirror the V2 runner's ``BlockTables`` on the host and flag its dummy mappings."""
    _track_instances(cls, REG.v2, _mirror_tables)

    def wrap_append(orig):
        def append_block_ids(self, req_index, new_block_ids, overwrite):
            starts = [0 if overwrite else int(self.num_blocks.np[g, req_index])
                      for g in range(self.num_kv_cache_groups)]
            orig(self, req_index, new_block_ids, overwrite)
            for g, start in enumerate(starts):
                ids = list(new_block_ids[g])
                if getattr(self, "redirect_writes_to_null_block", False):
                    ids = [0] * len(ids)
                self._echokv_host[g][req_index, start : start + len(ids)] = ids
        return append_block_ids
    _patch(cls, "append_block_ids", wrap_append)

    def flagging(dummy: bool):
        def wrap(orig):
            def method(self, *args, **kwargs):
                self._echokv_dummy = dummy
                return orig(self, *args, **kwargs)
            return method
        return wrap
    _patch(cls, "compute_slot_mappings", flagging(False))
    _patch(cls, "get_dummy_slot_mappings", flagging(True))


def install_v1_dummy(cls) -> None:
    """Count the V1 runner's ``_dummy_run`` frames: their steps use the device copy."""
    def wrap(orig):
        def _dummy_run(self, *args, **kwargs):
            REG.v1_dummy_depth += 1
            try:
                return orig(self, *args, **kwargs)
            finally:
                REG.v1_dummy_depth -= 1
        return _dummy_run
    _patch(cls, "_dummy_run", wrap)


def install() -> None:
    """Hook whichever of vLLM's block-table classes are importable (idempotent)."""
    try:
        from vllm.v1.worker.block_table import BlockTable
        from vllm.v1.worker.gpu_model_runner import GPUModelRunner

        _track_instances(BlockTable, REG.v1)
        install_v1_dummy(GPUModelRunner)
    except ImportError:
        pass
    try:
        from vllm.v1.worker.gpu.block_table import BlockTables

        install_v2(BlockTables)
    except ImportError:
        pass


def is_dummy_step(cm) -> bool:
    """Whether ``cm`` is one of vLLM's dummy steps (an all-PAD slot mapping)."""
    ptr = cm.block_table_tensor.data_ptr()
    if REG.v1_match(ptr) is not None:
        return REG.v1_dummy_depth > 0
    hit = REG.v2_match(ptr)
    return bool(hit and getattr(hit[0], "_echokv_dummy", False))


def _host_table(cm, block_size: int):
    """(host block table, batch row -> table row map or None), or None when the
    host copy cannot stand in for the device one."""
    ptr = cm.block_table_tensor.data_ptr()
    t = REG.v1_match(ptr)
    if t is not None:
        if (t.block_size != block_size or t.dcp_world_size != 1 or t.pcp_world_size != 1
                or REG.v1_dummy_depth):
            return None
        return t.block_table.np, None
    hit = REG.v2_match(ptr)
    if hit is not None:
        t, g = hit
        if (t.block_sizes[g] != block_size or t.cp_size != 1 or cm.req_idx is None
                or getattr(t, "_echokv_dummy", False)):
            return None
        return t._echokv_host[g], np.asarray(cm.req_idx, dtype=np.int64)
    return None


def host_lens_and_slots(cm, block_size: int):
    """``(seq_lens[:num_reqs], slot_mapping[:num_actual_tokens])`` as CPU int64 tensors,
    or None when they cannot be trusted (the caller then copies the device ones).
    Rows past the scheduled tokens (padding) map to -1, as on the device."""
    upper = cm.seq_lens_cpu_upper_bound
    if upper is None:
        return None
    found = _host_table(cm, block_size)
    if found is None:
        return None
    table, row_map = found
    n = cm.num_reqs
    starts = cm.query_start_loc_cpu[: n + 1].numpy().astype(np.int64)
    lens = upper[:n].numpy().astype(np.int64)
    total = int(starts[-1])
    if total > cm.num_actual_tokens:
        return None
    qlen = np.diff(starts)
    req = np.repeat(np.arange(n), qlen)                      # request of each token row
    pos = (lens - qlen)[req] + np.arange(total) - starts[:-1][req]  # its position in the sequence
    if row_map is not None and req.size and int(req.max()) >= row_map.size:
        return None
    rows = req if row_map is None else row_map[req]
    slots = np.full(cm.num_actual_tokens, -1, np.int64)
    slots[:total] = table[rows, pos // block_size].astype(np.int64) * block_size + pos % block_size
    return torch.from_numpy(lens), torch.from_numpy(slots)
