"""Per-block mixed-precision paged KV store inside a vLLM page budget.

Interface of ``echokv_vllm/tiered_cache.py`` (``NEXTRA`` 73, ``TieredLayout``
76-147, ``TieredKVCache`` 150-482). The page format is the stored-format
contract and is byte-identical to the reference:

    header   bs bytes: [0] tier (0 = never opened, else 2/4/8), [1] bitmask of
             K groups sealed early, [4:16] int32 ids of up to 3 pool chunks
    V stats  fp16 scale, fp16 min, each [bs, H, D / v_group]   (per token)
    K stats  fp16 scale, fp16 min, each [bs / k_group, H, D]   (per channel)
    data     mem_bits / 2 chunks of bs*H*D/2 bytes; token rows [K codes | V codes]

Chunk j of a block holds tokens [j*tpc, (j+1)*tpc), tpc = 2*bs/bits; chunk 0
is the block's own page, later chunks come from a per-layer pool of chunk
slots 1.. of every page (INT4 takes 1, INT8 takes 3). A block's tier is
fixed when offset 0 is written (forward-only), using the layer's tier then.

Host decisions (pool, demotion victims, counters) are native (``ChunkPool``
and ``WritePlanner`` wrap ``libechokv_host.so``); every device effect -- token
writes, K-group finalize, seal, demotion, reads -- is a HIP kernel of
``libechokv.so``, launched on the current stream. Page-header and residual-map updates are small index writes.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch
from torch.profiler import record_function

from echokv_amd import _host, _lib
from echokv_amd._util import to_device
from echokv_amd.write_plan import Eviction, SharedState, WriteMeta, WritePlan, stage_plan

SUPPORTED_BITS = (2, 4, 8)
NEXTRA = {2: 0, 4: 1, 8: 3}  # pool chunks a block needs beyond its own chunk 0


@dataclass(frozen=True)
class TieredLayout:
    num_kv_heads: int
    head_size: int
    block_size: int
    mem_bits: int
    k_group: int = 32
    v_group: int = 32

    def __post_init__(self) -> None:
        if self.mem_bits not in (2, 4, 6, 8):
            raise ValueError(f"mem_bits must be one of 2/4/6/8, got {self.mem_bits}")
        if self.block_size % 16 != 0:
            raise ValueError(f"block_size must be a multiple of 16, got {self.block_size}")
        if self.block_size % self.k_group != 0 or self.block_size // self.k_group > 8:
            raise ValueError(f"block_size {self.block_size} must be 1-8 multiples of k_group {self.k_group}")
        if self.head_size % self.v_group != 0 or self.head_size % 4 != 0:
            raise ValueError(f"head_size {self.head_size} must be divisible by v_group {self.v_group} and by 4")

    @staticmethod
    def per_token_bytes(num_kv_heads: int, head_size: int, mem_bits: int, k_group: int = 32,
                        v_group: int = 32) -> int:
        """Bytes per token vLLM must budget: header + stats + data, whole fp32 words."""
        h, d = num_kv_heads, head_size
        raw = 1 + 4 * h * (d // v_group) + 4 * h * d // k_group + (mem_bits // 2) * h * d // 2
        return -(-raw // 4) * 4

    @property
    def k_groups_per_block(self) -> int:
        return self.block_size // self.k_group

    @property
    def v_groups(self) -> int:
        return self.head_size // self.v_group

    @property
    def chunks_per_page(self) -> int:
        return self.mem_bits // 2

    @property
    def chunk_bytes(self) -> int:
        return self.block_size * self.num_kv_heads * self.head_size // 2

    @property
    def offsets(self) -> dict:
        bs, h, d = self.block_size, self.num_kv_heads, self.head_size
        vstat = bs * h * self.v_groups * 2
        kstat = self.k_groups_per_block * h * d * 2
        o = {"v_scale": bs, "v_min": bs + vstat, "k_scale": bs + 2 * vstat}
        o["k_min"] = o["k_scale"] + kstat
        o["data"] = o["k_min"] + kstat
        o["end"] = o["data"] + self.chunks_per_page * self.chunk_bytes
        return o

    @property
    def page_bytes(self) -> int:
        return self.offsets["end"]

    def side_bytes(self, bits: int) -> int:
        return self.num_kv_heads * self.head_size * bits // 8

    def row_bytes(self, bits: int) -> int:
        return 2 * self.side_bytes(bits)

    def tokens_per_chunk(self, bits: int) -> int:
        return 2 * self.block_size // bits

    # Decode streams each KV head's slice of every token row. The page header
    # (block_size bytes) puts the data field, like every other field, 16 bytes
    # past a 128-byte line when pages sit on 128-byte boundaries, and then half
    # the slices touch one line more. Pages placed `line_shift` bytes past a
    # 128-byte boundary have their data field on one: the same DMA pattern
    # streams about 1.27x faster on MI355X (93 -> 73 us for one INT4 layer).
    @property
    def line_shift(self) -> int:
        return -self.offsets["data"] % 128

    @property
    def aligned_stride(self) -> int:
        """A page stride, a multiple of 128 bytes, with room for ``line_shift``."""
        return -(-(self.page_bytes + self.line_shift) // 128) * 128

    def alloc_pages(self, num_blocks: int, device, zero: bool = False) -> torch.Tensor:
        """``[num_blocks, aligned_stride - line_shift]`` uint8 pages with every data field on a 128-byte line."""
        stride, shift = self.aligned_stride, self.line_shift
        buf = (torch.zeros if zero else torch.empty)(num_blocks * stride + 128, dtype=torch.uint8, device=device)
        start = -buf.data_ptr() % 128 + shift
        return buf.as_strided((num_blocks, stride - shift), (stride, 1), start)

    def abi(self, num_blocks: int, page_stride: int) -> _lib.Layout:
        o = self.offsets
        return _lib.Layout(self.num_kv_heads, self.head_size, self.block_size, self.k_group, self.v_group,
                           self.chunks_per_page, num_blocks, page_stride, o["v_scale"], o["v_min"], o["k_scale"],
                           o["k_min"], o["data"], self.chunk_bytes)


class ChunkPool:
    """Host side of one layer's store: the pool of extra chunks, each block's tier
    and chunk table, demotion victims and the per-tier counters, in native code
    (``ekh_pool_*``, ``echokv_amd/host/plan.cpp``) over the cache group's shared
    bookkeeping. The caller applies the device effects (demotion, headers)."""

    _COUNTERS = 23

    def __init__(self, layout: TieredLayout, num_blocks: int, shared: SharedState) -> None:
        lib = _host.lib()
        if shared.num_blocks != num_blocks:
            raise ValueError("shared state does not match this layer's cache")
        h = lib.ekh_pool_new(shared.planner._h, layout.chunks_per_page)
        if not h:
            raise ValueError(f"bad pool: {layout.chunks_per_page} chunks per page")
        self._h = C.c_void_p(h)
        self._free_fn = lib.ekh_pool_free
        self._planner = shared.planner  # keeps the bookkeeping the pool reads alive
        self.layout = layout
        self.n = num_blocks
        self.shared = shared
        self.tag_h = _host.view_i64(lib.ekh_pool_tags(self._h), num_blocks, self)

    def __del__(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._free_fn(h)
            self._h = None

    # -- counters ------------------------------------------------------------
    def _counters(self) -> np.ndarray:
        out = np.zeros(self._COUNTERS, np.int64)
        _host.lib().ekh_pool_counters(self._h, _host.i64p(out))
        return out

    @property
    def tokens_written(self) -> dict:
        c = self._counters()
        return {b: int(c[b]) for b in SUPPORTED_BITS}

    @property
    def blocks_opened(self) -> dict:
        c = self._counters()
        return {b: int(c[9 + b]) for b in SUPPORTED_BITS}

    @property
    def downgraded_blocks(self) -> int:
        return int(self._counters()[18])

    @property
    def demoted_blocks(self) -> int:
        return int(self._counters()[19])

    @property
    def sealed_groups(self) -> int:
        return int(self._counters()[20])

    @property
    def pool_size(self) -> int:
        return int(self._counters()[22])

    @property
    def free(self) -> list:
        """Free chunk ids, bottom to top (the last is handed out next)."""
        out = np.zeros(int(self._counters()[21]), np.int64)
        _host.lib().ekh_pool_free_list(self._h, _host.i64p(out), out.size)
        return out.tolist()

    def reset_counters(self) -> None:
        _host.lib().ekh_pool_reset_counters(self._h)

    # -- decisions -----------------------------------------------------------
    def open(self, blocks: np.ndarray, target_bits: int, protect, demote) -> tuple[np.ndarray, np.ndarray]:
        """(Re)open ``blocks`` at ``target_bits`` or the best tier the pool allows.

        When the pool runs short, ``demote(victims)`` is called with the least
        recently written full blocks the pool chose (never ``blocks`` or
        ``protect``) before the new headers exist. Returns ``(blocks, headers [n, 16])``."""
        blocks = _host.as_i64(blocks)
        prot = _host.as_i64(() if protect is None else protect)
        headers = np.zeros((blocks.size, 16), np.uint8)
        victims = np.zeros(self.n, np.int64)
        nv = C.c_int64(0)
        rc = _host.lib().ekh_pool_open(self._h, _host.i64p(blocks), blocks.size, int(target_bits), _host.i64p(prot),
                                       prot.size, headers.ctypes.data_as(_host.PU8), _host.i64p(victims),
                                       C.byref(nv))
        if rc != _host.OK:
            raise ValueError(f"cannot open blocks {blocks.tolist()[:8]} at {target_bits} bits")
        if nv.value:
            demote(victims[: nv.value].tolist())
        return blocks, headers

    def seal_row(self, ev: Eviction, planner=None) -> list[int]:
        """Device row (slot, block, group, fill, bits, mask) sealing ``ev``."""
        row = np.zeros(6, np.int64)
        e = np.array([ev.slot, ev.block, ev.group, ev.fill], np.int64)
        if _host.lib().ekh_pool_seal_row(self._h, _host.i64p(e), _host.i64p(row)) != _host.OK:
            raise ValueError(f"eviction of block {ev.block} is outside this pool")
        return row.tolist()

    def live_tiers(self) -> dict:
        """Blocks stored at each tier now (kept by the pool as blocks open and demote)."""
        out = np.zeros(9, np.int64)
        _host.lib().ekh_pool_live(self._h, _host.i64p(out))
        return {b: int(out[b]) for b in SUPPORTED_BITS}

    def majority_tier(self) -> int:
        """The tier most of the opened blocks are stored at (4 when nothing is open)."""
        live = self.live_tiers()
        best = max(SUPPORTED_BITS, key=lambda b: (live[b], b == 4))
        return best if live[best] else 4

    def fresh_opens(self, plan: WritePlan) -> np.ndarray:
        """Blocks to open this step: offset-0 writes plus writes into never-opened blocks."""
        opens = plan.open_np
        if plan.touched_np.size:
            fresh = plan.touched_np[self.tag_h[plan.touched_np] == 0]
            if fresh.size:
                opens = np.union1d(opens, fresh)
        return opens


class HeaderWriter:
    """The page headers of a step's opened blocks in every layer of a cache group
    (the same blocks open in every layer, each at its layer's tier), written by one
    launch (``echokv_write_headers``) instead of one index write per layer."""

    def __init__(self, stores) -> None:
        self.stores = list(stores)
        strides = {s.pages.stride(0) for s in self.stores}
        if len(strides) != 1:
            raise ValueError("the layers of one cache group must share the page stride")
        self.stride = strides.pop()
        self.num_blocks = min(s.pages.shape[0] for s in self.stores)
        bases = torch.tensor([s.pages.data_ptr() for s in self.stores], dtype=torch.int64)
        self.bases = to_device(bases, self.stores[0].device)

    def check(self, ids: np.ndarray) -> None:
        """Host check of the block ids before they go to the device."""
        if ids.size and (ids.min() < 0 or ids.max() >= self.num_blocks):
            raise ValueError(f"header block ids outside the {self.num_blocks} pages")

    def write(self, ids: torch.Tensor, headers: torch.Tensor) -> None:
        """``ids`` int64 ``[n]``; ``headers`` ``[n_layers * n * 16]`` bytes (any dtype view),
        layer-major, both on the device."""
        n = ids.numel()
        if headers.numel() * headers.element_size() != len(self.stores) * n * 16:
            raise ValueError("headers must hold 16 bytes per layer and block")
        _lib.call("echokv_write_headers", _lib.ptr(self.bases), len(self.stores), self.stride, _lib.ptr(ids), n,
                  _lib.ptr(headers), _lib.stream())


class TieredKVCache:
    """One layer's tiered store over ``pages``: a uint8 ``[num_blocks, >= page_bytes]`` device view."""

    def __init__(self, layout: TieredLayout, pages: torch.Tensor, residual_slots: int = 256,
                 residual_dtype: torch.dtype = torch.float32, residual: torch.Tensor | None = None,
                 shared: SharedState | None = None) -> None:
        if pages.dtype != torch.uint8 or pages.dim() != 2:
            raise ValueError("pages must be a 2-D uint8 tensor")
        if pages.shape[1] < layout.page_bytes:
            raise ValueError(f"page has {pages.shape[1]} bytes, layout needs {layout.page_bytes}")
        if pages.stride(1) != 1 or pages.stride(0) % 16 != 0:
            raise ValueError("pages must be byte-contiguous with a 16-byte aligned row stride")
        _lib.require_device(pages)
        L = layout
        n = pages.shape[0]
        h, d, bs = L.num_kv_heads, L.head_size, L.block_size
        o = L.offsets
        self.layout = L
        self.num_blocks = n
        self.device = pages.device
        self.pages = pages
        self.header = pages[:, :16]
        self.tag = pages[:, 0]
        self.sealed = pages[:, 1]
        self.table = pages[:, 4:16].view(torch.int32)

        def f16(name, nxt, *shape):
            return pages[:, o[name] : o[nxt]].view(torch.float16).view(n, *shape)

        self.v_scale = f16("v_scale", "v_min", bs, h, L.v_groups)
        self.v_min = f16("v_min", "k_scale", bs, h, L.v_groups)
        self.k_scale = f16("k_scale", "k_min", L.k_groups_per_block, h, d)
        self.k_min = f16("k_min", "data", L.k_groups_per_block, h, d)
        self.data = pages[:, o["data"] : o["end"]].view(n, L.chunks_per_page, L.chunk_bytes)
        pages[:, :bs].zero_()

        if residual is None:
            residual = torch.zeros(residual_slots + 1, L.k_group, h, d, dtype=residual_dtype, device=self.device)
        if residual.shape[1:] != (L.k_group, h, d) or residual.shape[0] < 2:
            raise ValueError(f"residual buffer shape {tuple(residual.shape)} does not match layout")
        r = residual.shape[0] - 1
        if shared is None:
            shared = SharedState(n, bs, L.k_group, r, kref_window=L.k_group, device=self.device)
        if shared.num_blocks != n or shared.planner.num_slots > r:
            raise ValueError("shared state does not match this layer's cache")
        self.shared = shared
        self.res_k = residual
        self.res_group = shared.res_group
        self.block_res = shared.block_res
        self.planner = shared.planner
        self.pool = ChunkPool(L, n, shared)
        self.abi = L.abi(n, pages.stride(0))

    # -- counters (tiered_cache.py:228-254) -------------------------------------
    @property
    def tokens_written(self) -> dict:
        return self.pool.tokens_written

    def reset_counters(self) -> None:
        self.pool.reset_counters()

    @property
    def pool_size(self) -> int:
        return self.pool.pool_size

    @property
    def pool_free(self) -> int:
        return int(self.pool._counters()[21])

    @property
    def residual_free(self) -> int:
        return len(self.planner.free)

    @property
    def blocks_opened(self) -> dict:
        return self.pool.blocks_opened

    @property
    def downgraded_blocks(self) -> int:
        return self.pool.downgraded_blocks

    @property
    def demoted_blocks(self) -> int:
        return self.pool.demoted_blocks

    @property
    def sealed_groups(self) -> int:
        return self.pool.sealed_groups

    @property
    def _tag_h(self) -> np.ndarray:
        return self.pool.tag_h

    # -- host decisions + their device effects ----------------------------------
    def open_blocks(self, blocks, target_bits: int, protect=None) -> tuple[np.ndarray, np.ndarray]:
        """(Re)open ``blocks`` at ``target_bits`` or the best tier that fits; returns
        ``(blocks, headers)`` for ``write_headers`` (``tiered_cache.py:258-303``)."""
        if target_bits not in SUPPORTED_BITS:
            raise ValueError(f"unsupported target bits {target_bits}")
        blocks = np.asarray(blocks.cpu() if torch.is_tensor(blocks) else blocks, dtype=np.int64)
        return self.pool.open(blocks, target_bits, protect, self._demote)

    def write_headers(self, blocks: torch.Tensor, headers: torch.Tensor) -> None:
        self.header[blocks] = headers

    def _demote(self, victims: list[int]) -> None:
        """Requantize whole blocks to INT2 in place (``tiered_cache.py:309-346``):
        dequantize at their current tiers (HIP gather), then requantize (HIP store)."""
        L = self.layout
        vb = to_device(torch.tensor(victims, dtype=torch.int64), self.device)
        blk = vb.repeat_interleave(L.block_size)
        off = torch.arange(L.block_size, device=self.device).repeat(len(victims))
        k, v = self.gather(blk, off)
        _lib.call("echokv_store_blocks", _lib.byref(self.abi), _lib.ptr(self.pages), _lib.ptr(vb), len(victims),
                  _lib.ptr(k), _lib.ptr(v), 2, _lib.stream())

    def _seal_rows(self, rows: list) -> None:
        self.seal_groups(to_device(torch.tensor(rows, dtype=torch.int64).reshape(-1, 6), self.device))

    def seal_groups(self, rows: torch.Tensor) -> None:
        """Seal evicted residual groups: ``rows`` int64 ``[n, 6]`` on the device, as
        ``ChunkPool.seal_row`` makes them (``tiered_cache.py:379-394``)."""
        if rows.dtype != torch.int64 or rows.dim() != 2 or rows.shape[1] != 6 or rows.stride(1) != 1:
            raise ValueError("seal rows must be int64 [n, 6] with contiguous rows")
        if rows.shape[0] == 0:
            return
        res = _lib.residual(self.res_k)
        _lib.call("echokv_seal_groups", _lib.byref(self.abi), _lib.ptr(self.pages), _lib.ptr(rows), rows.shape[0],
                  _lib.byref(res), _lib.stream())

    def _seal(self, ev: Eviction) -> None:
        if ev.fill > 0:
            self._seal_rows([self.pool.seal_row(ev, self.planner)])

    def prepare(self, plan: WritePlan, target_bits: int):
        """Host side of a step's writes: seal evicted groups, open blocks (``tiered_cache.py:396-413``)."""
        rows = [self.pool.seal_row(e, self.planner) for e in plan.evictions if e.fill > 0]
        if rows:
            self._seal_rows(rows)
        opens = self.pool.fresh_opens(plan)
        if not opens.size:
            return None
        return self.open_blocks(opens, target_bits, protect=plan.touched_np)

    def apply(self, meta: WriteMeta, key: torch.Tensor, value: torch.Tensor, kref: torch.Tensor | None = None,
              capturing: bool = False) -> None:
        """Device side: finalize completed K groups, then store the step's tokens
        (``tiered_cache.py:415-432``), as one launch. ``capturing`` launches full
        grids masked by the device counts, as a replayed graph needs."""
        from echokv_amd.kernels.write import FUSED_MAX_K_GROUP, finalize_k, write_step, write_tokens

        # The reference's scopes (tiered_cache.py:428,431): one launch here does the
        # work of both, so it is recorded under both names, nested.
        if self.layout.k_group <= FUSED_MAX_K_GROUP:
            with record_function("echokv.write.k_finalize"), record_function("echokv.write.tokens"):
                write_step(self, key, value, meta, kref, full_grid=capturing)
            return
        if capturing or meta.n_fin:
            with record_function("echokv.write.k_finalize"):
                finalize_k(self, key, meta, full_grid=capturing)
        if meta.n_rows:
            with record_function("echokv.write.tokens"):
                write_tokens(self, key, value, meta, kref)

    def write(self, key: torch.Tensor, value: torch.Tensor, slots: torch.Tensor, target_bits: int,
              kref: torch.Tensor | None = None) -> None:
        """Standalone path: plan, prepare and apply in one call (``tiered_cache.py:434-447``)."""
        plan = self.planner.plan(slots.detach().cpu())
        opened = self.prepare(plan, target_bits)
        self.shared.commit(plan)
        meta, extra = stage_plan(plan, self.device, opened)
        self.shared.apply_res_map(*extra[:4])
        if opened is not None:
            self.write_headers(extra[4], extra[5])
        self.apply(meta, key, value, kref)

    # -- read ----------------------------------------------------------------------
    def gather(self, blk: torch.Tensor, off: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Dequantized K and V (float32 ``[n, H, D]``) of tokens (blk, off) (``tiered_cache.py:451-478``)."""
        L = self.layout
        blk = blk.to(device=self.device, dtype=torch.int64).contiguous()
        off = off.to(device=self.device, dtype=torch.int64).contiguous()
        n = blk.numel()
        k = torch.empty(n, L.num_kv_heads, L.head_size, device=self.device)
        v = torch.empty_like(k)
        res = _lib.residual(self.res_k)
        _lib.call("echokv_gather", _lib.byref(self.abi), _lib.ptr(self.pages), _lib.ptr(self.block_res),
                  _lib.ptr(self.res_group), _lib.byref(res), _lib.ptr(blk), _lib.ptr(off), n, _lib.ptr(k), _lib.ptr(v),
                  _lib.stream())
        return k, v

    def tier_histogram(self) -> dict:
        return {b: int((self.tag == b).sum()) for b in SUPPORTED_BITS}

