"""vLLM's slot mapping and sequence lengths, computed on the host.

Interface of ``echokv_vllm/host_slots.py`` (``install``, ``install_v2``,
``install_v1_dummy``, ``is_dummy_step``, ``host_lens_and_slots``).

Why: vLLM builds ``slot_mapping`` on the device. The write planner needs it on
the host, and reading the device copy would wait for the previous step to
drain, so the host could no longer prepare step N+1 while the GPU runs step N.
The mapping is a pure function of host-side facts vLLM already has:

* each token's position, from ``query_start_loc_cpu`` and
  ``seq_lens_cpu_upper_bound`` (exact unless asynchronous speculative decoding
  is on, in which case the builder does not use this module);
* each position's block id, from a host copy of the block table. vLLM's V1
  runner keeps one (``BlockTable.block_table.np``, indexed by batch row); its
  V2 runner keeps tables on the device only (indexed by request slot, written
  through ``BlockTables.append_block_ids``), so this module keeps a host mirror
  of those writes and maps batch rows to slots with ``cm.req_idx``.

The arithmetic (``slot = table[row][pos // bs] * bs + pos % bs``) runs in native
code (``ekh_host_slots``). Each step's ``block_table_tensor`` is matched to its
host source by the device tensor's address, through a registry filled when the
vLLM objects are built.

Dummy steps (warm-up, profiling, graph capture, idle data-parallel ranks) write
nothing -- their device mapping is all -1 -- while their table rows may still
name live requests' blocks. They are recognised (V1: a ``_dummy_run`` is on the
stack; V2: the runner last asked for dummy slot mappings) and left to the
device copy.
"""

from __future__ import annotations

import ctypes as C
import functools
import weakref

import numpy as np
import torch

from echokv_amd import _host

_HOOKED = "__echokv_hooked__"


class _Source:
    """One host table that stands in for one device block table."""

    __slots__ = ("owner", "kind", "group")

    def __init__(self, owner, kind: str, group: int) -> None:
        self.owner = weakref.ref(owner)
        self.kind = kind  # "v1" or "v2"
        self.group = group


class _Registry:
    """Device block-table address -> its host source, plus the V1 dummy-run depth."""

    def __init__(self) -> None:
        self.sources: dict[int, _Source] = {}
        self.v1_dummy_runs = 0

    def add(self, ptr: int, owner, kind: str, group: int = 0) -> None:
        self.sources[ptr] = _Source(owner, kind, group)

    def find(self, ptr: int):
        """``(owner, kind, group)`` of the live source registered at ``ptr``, else None."""
        src = self.sources.get(ptr)
        if src is None:
            return None
        owner = src.owner()
        if owner is None:  # collected: its address may be reused by an unrelated tensor
            del self.sources[ptr]
            return None
        return owner, src.kind, src.group


REGISTRY = _Registry()


def _hook(cls, name: str, make):
    """Wrap ``cls.name`` with ``make(original)`` once (installing twice is a no-op)."""
    orig = getattr(cls, name)
    if getattr(orig, _HOOKED, False):
        return
    wrapped = functools.wraps(orig)(make(orig))
    setattr(wrapped, _HOOKED, True)
    setattr(cls, name, wrapped)


def _after_init(cls, register) -> None:
    def make(init):
        def __init__(self, *args, **kwargs):
            init(self, *args, **kwargs)
            register(self)
        return __init__
    _hook(cls, "__init__", make)


# ---- V1 runner -------------------------------------------------------------------

def _register_v1(table) -> None:
    REGISTRY.add(table.block_table.gpu.data_ptr(), table, "v1")


def install_v1_dummy(cls) -> None:
    """Count the V1 runner's ``_dummy_run`` frames: steps inside one are dummy steps."""
    def make(run):
        def _dummy_run(self, *args, **kwargs):
            REGISTRY.v1_dummy_runs += 1
            try:
                return run(self, *args, **kwargs)
            finally:
                REGISTRY.v1_dummy_runs -= 1
        return _dummy_run
    _hook(cls, "_dummy_run", make)


def install_v1(table_cls, runner_cls=None) -> None:
    _after_init(table_cls, _register_v1)
    if runner_cls is not None:
        install_v1_dummy(runner_cls)


# ---- V2 runner -------------------------------------------------------------------

def _register_v2(tables) -> None:
    # The host mirror of every device table (int32, as V1's host copy).
    tables._echokv_mirror = [np.zeros(tuple(t.gpu.shape), np.int32) for t in tables.block_tables]
    tables._echokv_dummy_map = False
    for g, inp in enumerate(tables.input_block_tables):
        REGISTRY.add(inp.data_ptr(), tables, "v2", g)


def install_v2(cls) -> None:
    """Mirror a V2 ``BlockTables``' writes on the host and flag its dummy slot mappings."""
    _after_init(cls, _register_v2)

    def make_append(append):
        def append_block_ids(self, req_index, new_block_ids, overwrite):
            # Where each group's ids land: vLLM appends after the request's current
            # blocks unless it overwrites the row (a slot reused by a new request).
            at = [0 if overwrite else int(self.num_blocks.np[g, req_index]) for g in range(self.num_kv_cache_groups)]
            append(self, req_index, new_block_ids, overwrite)
            null = getattr(self, "redirect_writes_to_null_block", False)
            for g, start in enumerate(at):
                ids = np.asarray(new_block_ids[g], np.int32)
                self._echokv_mirror[g][req_index, start : start + ids.size] = 0 if null else ids
        return append_block_ids
    _hook(cls, "append_block_ids", make_append)

    def flag(dummy: bool):
        def make(method):
            def flagged(self, *args, **kwargs):
                self._echokv_dummy_map = dummy
                return method(self, *args, **kwargs)
            return flagged
        return make
    _hook(cls, "compute_slot_mappings", flag(False))
    _hook(cls, "get_dummy_slot_mappings", flag(True))


def install() -> None:
    """Hook whichever of vLLM's block-table classes are importable (idempotent)."""
    try:
        from vllm.v1.worker.block_table import BlockTable
        from vllm.v1.worker.gpu_model_runner import GPUModelRunner

        install_v1(BlockTable, GPUModelRunner)
    except ImportError:
        pass
    try:
        from vllm.v1.worker.gpu.block_table import BlockTables

        install_v2(BlockTables)
    except ImportError:
        pass


# ---- per step --------------------------------------------------------------------

def is_dummy_step(cm) -> bool:
    """Whether ``cm`` belongs to one of vLLM's dummy steps (an all-PAD slot mapping)."""
    hit = REGISTRY.find(cm.block_table_tensor.data_ptr())
    if hit is None:
        return False
    owner, kind, _ = hit
    return REGISTRY.v1_dummy_runs > 0 if kind == "v1" else bool(owner._echokv_dummy_map)


def _host_table(cm, block_size: int):
    """``(int32 host table, batch row -> table row or None)`` standing in for ``cm``'s
    device table, or None when it cannot (unknown table, another block size,
    context parallelism, a dummy step, V2 without ``req_idx``)."""
    hit = REGISTRY.find(cm.block_table_tensor.data_ptr())
    if hit is None:
        return None
    owner, kind, g = hit
    if kind == "v1":
        usable = (owner.block_size == block_size and owner.dcp_world_size == 1 and owner.pcp_world_size == 1
                  and REGISTRY.v1_dummy_runs == 0)
        return (owner.block_table.np, None) if usable else None
    if owner.block_sizes[g] != block_size or owner.cp_size != 1 or cm.req_idx is None or owner._echokv_dummy_map:
        return None
    return owner._echokv_mirror[g], np.asarray(cm.req_idx, dtype=np.int64)


def host_lens_and_slots(cm, block_size: int):
    """``(seq_lens[:num_reqs], slot_mapping[:num_actual_tokens])`` as CPU int64 tensors,
    or None when the host copies cannot be trusted (the caller then copies the device
    ones). Token rows past the scheduled ones (padding) map to -1, as on the device."""
    upper = cm.seq_lens_cpu_upper_bound
    if upper is None:
        return None
    found = _host_table(cm, block_size)
    if found is None:
        return None
    table, row_map = found
    n, t = cm.num_reqs, cm.num_actual_tokens
    qsl = np.ascontiguousarray(cm.query_start_loc_cpu[: n + 1].numpy(), dtype=np.int32)
    lens = np.ascontiguousarray(upper[:n].numpy(), dtype=np.int32)
    if table.dtype != np.int32 or table.ndim != 2 or table.strides[1] != 4:
        table = np.ascontiguousarray(table, dtype=np.int32)
    slots = np.empty(t, np.int64)
    batch = _host.Batch(n, t, qsl.ctypes.data, lens.ctypes.data, None)
    rm = None if row_map is None else np.ascontiguousarray(row_map, dtype=np.int64)
    rc = _host.lib().ekh_host_slots(C.byref(batch), table.ctypes.data, table.shape[0], table.shape[1],
                                    table.strides[0] // 4, None if rm is None else rm.ctypes.data,
                                    0 if rm is None else rm.size, block_size, slots.ctypes.data)
    if rc != _host.OK:
        return None
    return torch.from_numpy(lens.astype(np.int64)), torch.from_numpy(slots)
