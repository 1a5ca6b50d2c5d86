"""vLLM attention backend ("CUSTOM") over the MI355X tiered KV store.

Interface of ``echokv_vllm/backend.py:72-636``: ``EchoKVAttentionBackend``
(``customize_spec``, block / head-size support, ``get_name() == "CUSTOM"``),
``EchoKVMetadataBuilder`` (``build`` once per step for every layer) and
``EchoKVAttentionImpl`` (``bind``, ``do_kv_cache_update``, ``forward``). vLLM
budgets the page as one opaque byte state per token (``customize_spec``), so its
cache manager, memory profiler and block tables see exactly the bytes the tiered
store uses.

How a step runs here:

* ``build`` makes every host decision of the step for all layers in one native
  call (``StepDriver``, ``echokv_amd/step.py``): the batch layout, the write plan,
  the blocks that open in each layer at that layer's tier, and the canary rows.
  One host-to-device copy then carries the step's metadata; the few device
  effects that must precede the layers' writes (residual-map and page-header
  updates, and the rare seals and demotions) are launched right away.
* The canary has its own clock (``CanaryClock``): a fire step stashes query rows,
  the next build scores every layer at once and hands each controller the
  previous fire's δ̂, which the GPU finished long ago, so reading it never waits.
* ``do_kv_cache_update`` and ``forward`` only launch HIP kernels on device
  metadata (``WriteMeta``, ``DecodeWork``, ``PrefillWork``), so a decode-only step
  replays as one HIP graph.

The torch-profiler scopes are the reference's (``echokv.build``,
``echokv.canary``, ``echokv.write``, ``echokv.prefill_attn``,
``echokv.decode_attn``; inside ``echokv.write`` the store's ``echokv.write.k_finalize``
and ``echokv.write.tokens``), so the reference's
profiling harness reads the same report. There is no other path: without the HIP
library every call raises.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, replace
from typing import ClassVar

import numpy as np
import torch
from torch.profiler import record_function

from echokv_amd import _vllm
from echokv_amd._vllm import (
    AttentionBackend,
    AttentionCGSupport,
    AttentionImpl,
    AttentionMetadataBuilder,
    AttentionType,
    MultipleOf,
)
from echokv_amd.canary import canary_kl, ring_view
from echokv_amd.config import load_config, v_group_supported
from echokv_amd.controller import SUPPORTED_BITS, LayerController
from echokv_amd.host_slots import host_lens_and_slots, is_dummy_step
from echokv_amd.kernels import decode as dec
from echokv_amd.kernels import prefill as pf
from echokv_amd.step import StepDriver
from echokv_amd.tiered_cache import HeaderWriter, TieredKVCache, TieredLayout
from echokv_amd.write_plan import SharedState, WriteMeta

# Head sizes the MFMA kernels take (decode at 256 as two 128-channel half-heads,
# prefill at 256 on the fused kernel alone); others up to MAX_HEAD_SIZE take the
# fp32 kernels.
KERNEL_HEAD_SIZES = (64, 128, 256)
MAX_HEAD_SIZE = 256
# Upper bound on decode splits per sequence (a fixed grid, so a graph replays it).
MAX_DECODE_SPLITS = dec.MAX_SPLITS


class EchoKVAttentionBackend(AttentionBackend):
    forward_includes_kv_cache_update: bool = False

    supported_dtypes: ClassVar[list[torch.dtype]] = [torch.float16, torch.bfloat16, torch.float32]
    supported_kv_cache_dtypes: ClassVar[list[str]] = ["auto", "float16", "bfloat16"]

    @classmethod
    def customize_spec(cls, spec):
        """One opaque state of ``per_token_bytes`` per token and block slot."""
        cfg = load_config()
        if getattr(spec, "head_size_v", spec.head_size) != spec.head_size:
            raise NotImplementedError("EchoKV requires head_size_v == head_size")
        per_token = TieredLayout.per_token_bytes(spec.num_kv_heads, spec.head_size, cfg.mem_bits, cfg.k_group,
                                                 cfg.v_group)
        return replace(spec, num_head_slots=1, state_content_bytes=per_token)

    @staticmethod
    def get_supported_kernel_block_sizes(kv_cache_spec=None) -> list:
        return [MultipleOf(block_multiple())]

    @classmethod
    def supports_block_size(cls, block_size: int | None) -> bool:
        return block_size is None or block_size % block_multiple() == 0

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        """The reference's rule (a multiple of 4 and of the V group) up to 256
        channels, for V groups the kernels store (``v_group_supported``)."""
        vg = load_config().v_group
        return head_size % 4 == 0 and head_size <= MAX_HEAD_SIZE and v_group_supported(vg, head_size)

    @classmethod
    def supports_attn_type(cls, attn_type: str) -> bool:
        return attn_type == AttentionType.DECODER

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls():
        return EchoKVAttentionImpl

    @staticmethod
    def get_builder_cls():
        return EchoKVMetadataBuilder


def block_multiple() -> int:
    """Block sizes must be multiples of this (a block holds whole K groups)."""
    return max(16, load_config().k_group)


# ---- per-step device work --------------------------------------------------------

@dataclass
class DecodeWork:
    """One decode entry per single-token request (graph padding: length 0)."""

    rows: torch.Tensor  # query rows
    reqs: torch.Tensor  # block-table rows
    lens: torch.Tensor  # cache lengths, the new token included
    num_splits: int  # split grid (fixed, so a graph replays it)
    workspace: tuple | None  # (acc, ml) shared by every layer; None: the call allocates
    batch_invariant: bool
    tier_masks: torch.Tensor | None = None  # [layers, 2] int32: each layer's live tiers, read by the kernels
    host_tier_masks: np.ndarray | None = None  # [layers] the same, on the host

    def run(self, impl, query: torch.Tensor, block_table: torch.Tensor, out: torch.Tensor) -> None:
        # Each tier the layer holds runs on its own fast path (tier passes, on the
        # split schedule): under graph capture through the device mask (read when the
        # kernels run, so a replayed graph follows the layer's tiers); eagerly, a layer
        # holding one tier runs that tier's kernel alone, and one holding several
        # takes the tier passes on either schedule (the balanced kernel has none: its
        # other tiers' blocks would take the generic path, about 2.6x slower a block).
        tier, mask, inv, ws = impl.decode_tier(), None, self.batch_invariant, self.workspace
        if self.tier_masks is not None:
            if _capturing(query):
                if inv:
                    mask = self.tier_masks[impl.group_index, :1]
            else:
                held = int(self.host_tier_masks[impl.group_index])
                if held & (held - 1):
                    mask = self.tier_masks[impl.group_index, :1]
                    if not inv:
                        inv = True
                        ws = impl.split_workspace(ws, self.lens.shape[0], self.num_splits)
                elif held:
                    tier = held
        dec.decode_attention(impl.store, query, block_table, self.lens, impl.scale, q_rows=self.rows,
                             bt_rows=self.reqs, out=out, num_splits=self.num_splits, workspace=ws,
                             tier=tier, batch_invariant=inv, tier_mask=mask)


@dataclass
class PrefillWork:
    """The step's prefill chunks and the device tables of the path that runs them."""

    entries: list  # (q_start, q_end, context, 0) per chunk
    reqs: list  # block-table row of each chunk
    tiles: torch.Tensor | None = None  # fused path (every chunk <= 64 tokens)
    dense: tuple | None = None  # (DensePlan, workspace) of the two-pass path
    own_group_rows: torch.Tensor | None = None  # own-group-exact prefill (ECHOKV_OWN_GROUP_EXACT=1)

    def run(self, impl, query: torch.Tensor, key: torch.Tensor, block_table: torch.Tensor,
            out: torch.Tensor) -> None:
        og_key = None
        if self.own_group_rows is not None:  # each query's own K group from this step's key rows
            og_key = key.view(key.shape[0], impl.num_kv_heads, impl.head_size)
        pf.prefill_attention(impl.store, query, out, self.entries, self.reqs, block_table, impl.scale,
                             tiles=self.tiles, dense=self.dense, own_group_key=og_key,
                             own_group_rows=self.own_group_rows)


@dataclass
class EchoKVMetadata:
    num_actual_tokens: int
    num_reqs: int
    query_start_loc_cpu: torch.Tensor
    seq_lens_cpu: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    write: WriteMeta | None  # None: no KV cache bound yet (memory profiling); attention is skipped
    decode: DecodeWork | None = None
    prefill: PrefillWork | None = None
    canary_rows: torch.Tensor | None = None  # [canary_max_q] query rows the canary reads
    fire: bool = False  # this step's query rows feed the canary (scored at the next build)


# ---- canary schedule ---------------------------------------------------------------

class CanaryClock:
    """When the canary fires and when its result reaches the controllers.

    Every ``interval``-th real step arms the clock; the next step with a live
    request fires: its newest query rows are stashed by ``forward``. The build
    after a fire scores every layer from the stash (``echokv.canary``) and feeds
    the controllers the fire before it, so reading δ̂ back never waits for the
    GPU (the reference's schedule, ``echokv_vllm/backend.py:314-333,395-408``).
    """

    def __init__(self, interval: int) -> None:
        self.interval = interval
        self.steps = 0
        self.armed = False
        self.stashed: tuple | None = None  # (rows, mean context) of the last fire, not yet scored
        self.scored: tuple | None = None  # (δ̂ [layers, tiers] on the device, mean context), not yet fed

    def tick(self, dummy: bool) -> bool:
        """Count a step; whether this step should take canary rows."""
        if not dummy:
            self.steps += 1
            if self.steps % self.interval == 0:
                self.armed = True
        return self.armed

    def fired(self, rows: int, ctx: float) -> None:
        if rows:
            self.armed = False
            self.stashed = (rows, ctx)

    def reset(self) -> None:
        self.stashed = self.scored = None


# ---- builder -------------------------------------------------------------------------

class _Group:
    """A cache group's layers once bound to their KV caches: stores, shared state,
    the step driver, header writer and shared canary workspace."""

    def __init__(self, builder, layers: list, caches: list) -> None:
        cfg = builder.cfg
        self.impls = [layer.impl for layer in layers]
        self.shared = SharedState(caches[0].shape[0], builder.kv_cache_spec.block_size, cfg.k_group,
                                  builder.residual_slots, cfg.kref_window, builder.device)
        for i, (impl, cache) in enumerate(zip(self.impls, caches)):
            impl.bind(cache, self.shared)
            impl.group_index = i  # this layer's row of the step's per-layer device tables
        self.stores = [impl.store for impl in self.impls]
        self.driver = StepDriver(self.shared, self.stores, builder.cap, cfg.canary_max_q, builder.device)
        self.headers = HeaderWriter(self.stores)
        impl0 = self.impls[0]
        self.canary_ws = torch.empty(len(self.impls) * impl0.num_kv_heads * len(SUPPORTED_BITS),
                                     device=impl0.store.device)
        self.cache_ptr = caches[0].data_ptr()

    def tiers(self) -> np.ndarray:
        return np.fromiter((impl.controller.bits for impl in self.impls), np.int32, len(self.impls))


class EchoKVMetadataBuilder(AttentionMetadataBuilder):
    _cudagraph_support: ClassVar = AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE

    @classmethod
    def get_cudagraph_support(cls, vllm_config, kv_cache_spec):
        """Decode-only batches replay a full graph: ``build`` makes every host decision
        and ``forward`` only launches kernels. ``ECHOKV_CUDAGRAPH=0`` turns that off."""
        bs = kv_cache_spec.block_size
        if os.environ.get("ECHOKV_CUDAGRAPH", "1") != "1" or bs & (bs - 1):
            return AttentionCGSupport.NEVER
        return cls._cudagraph_support

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device) -> None:
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        self.cfg = load_config()
        self.gqa = _vllm.num_attention_heads(vllm_config, layer_names) // kv_cache_spec.num_kv_heads
        # Exact host sequence lengths are not available under async speculative decoding.
        self.host_slots = getattr(vllm_config, "speculative_config", None) is None
        self.check_host_slots = os.environ.get("ECHOKV_CHECK_HOST_SLOTS", "0") == "1"
        self.host_slot_steps = 0
        self.num_splits = decode_splits(vllm_config.model_config.max_model_len, kv_cache_spec.block_size)
        self.residual_slots = residual_slots(self.cfg, vllm_config)
        self.cap = graph_capacity(vllm_config)
        self.layers: list | None = None  # bind_layers (standalone drivers) or vLLM's layers
        self.group: _Group | None = None
        self.canary = CanaryClock(self.cfg.canary_interval)

    @property
    def shared(self) -> SharedState | None:
        return None if self.group is None else self.group.shared

    def bind_layers(self, layers: list) -> None:
        """The attention layers of this group (objects with ``kv_cache`` and ``impl``)."""
        self.layers = list(layers)
        self.group = None

    def _bound(self) -> _Group | None:
        """The group over the layers' current caches; None while vLLM profiles memory
        (no KV cache yet). Rebinds when vLLM hands the layers new caches."""
        if self.layers is None:
            self.layers = _vllm.attention_layers(self.vllm_config, self.layer_names)
        caches = [getattr(layer, "kv_cache", None) for layer in self.layers]
        if not caches or any(c is None or c.numel() == 0 for c in caches):
            return None
        if self.group is None or self.group.cache_ptr != caches[0].data_ptr():
            self.group = _Group(self, self.layers, caches)
            self.canary.reset()
        return self.group

    # -- the step ---------------------------------------------------------------
    def build(self, common_prefix_len: int, common_attn_metadata, fast_build: bool = False) -> EchoKVMetadata:
        with record_function("echokv.build"):
            return self._build(common_attn_metadata)

    def _mapping(self, cm, dummy: bool):
        """The step's (lengths, slots) on the host: derived from host copies when vLLM
        exposes them, else read back from the device (a wait: dummy steps only)."""
        bs = self.kv_cache_spec.block_size
        n, t = cm.num_reqs, cm.num_actual_tokens
        host = host_lens_and_slots(cm, bs) if self.host_slots else None
        if host is not None:
            self.host_slot_steps += 1
            if not self.check_host_slots:
                return host
        elif self.check_host_slots and self.host_slots and not dummy:
            raise AssertionError("ECHOKV_CHECK_HOST_SLOTS=1 but the host slot mapping is unavailable")
        dev = (cm.seq_lens[:n].cpu().long(), cm.slot_mapping[:t].cpu().long())
        if host is not None and not (torch.equal(host[0], dev[0]) and torch.equal(host[1], dev[1])):
            raise AssertionError("EchoKV host slot mapping differs from vLLM's")
        return dev

    def _build(self, cm) -> EchoKVMetadata:
        if getattr(cm, "causal", True) is not True:
            raise NotImplementedError("EchoKV supports causal decoder attention only")
        n, t = cm.num_reqs, cm.num_actual_tokens
        dummy = is_dummy_step(cm)
        lens, slots = self._mapping(cm, dummy)
        md = EchoKVMetadata(num_actual_tokens=t, num_reqs=n, query_start_loc_cpu=cm.query_start_loc_cpu[: n + 1],
                            seq_lens_cpu=lens, block_table=cm.block_table_tensor, slot_mapping=cm.slot_mapping,
                            write=None)
        group = self._bound()
        if group is None:
            return md
        if self.canary.stashed is not None:
            self._score_canary(group)  # before this step's writes move the K_ref ring
        fire = self.canary.tick(dummy)
        qsl = np.ascontiguousarray(cm.query_start_loc_cpu[: n + 1].numpy(), dtype=np.int32)
        up = group.driver.run(qsl, np.ascontiguousarray(lens.numpy(), dtype=np.int32),
                              np.ascontiguousarray(slots.numpy(), dtype=np.int64), group.tiers(), fire)
        self.canary.fired(up.n_canary, up.canary_ctx)
        group.driver.apply(up, group.headers)
        md.write = WriteMeta(tok=up.tok, fin=up.fin, fin_count=up.fin_count, n_rows=up.n_tokens, n_fin=up.n_fin)
        md.canary_rows = up.canary_rows
        md.fire = up.n_canary > 0
        if up.decode is not None:
            n_dec = up.decode[0].numel()
            md.decode = DecodeWork(*up.decode, num_splits=self.num_splits, tier_masks=up.tier_masks,
                                   host_tier_masks=up.host_tier_masks,
                                   workspace=group.impls[0].decode_workspace(n_dec, self.num_splits, self.cap),
                                   batch_invariant=self.cfg.batch_invariant)
        if up.prefill:
            md.prefill = self._prefill_work(group, up.prefill)
        return md

    def _prefill_work(self, group: _Group, chunks: list) -> PrefillWork:
        entries = [(qs, qe, ctx, 0) for qs, qe, ctx, _ in chunks]
        work = PrefillWork(entries=entries, reqs=[r for *_, r in chunks])
        impl0 = group.impls[0]
        dev = self.device
        if pf.kernels_take(impl0.head_size, self.gqa):
            if not pf.use_dense(entries, impl0.head_size):
                work.tiles = pf.build_tiles(entries, work.reqs, self.gqa, dev,
                                            tokens=pf.block_m(self.gqa, impl0.head_size))
            else:
                plan = pf.build_dense_plan(entries, work.reqs, self.gqa, dev)
                nbytes = pf.dense_workspace_bytes(impl0.store, plan.packs.shape[0])
                work.dense = (plan, torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev))
        if self.cfg.own_group_exact:
            work.own_group_rows = pf.build_own_group_rows(entries, work.reqs, dev)
        return work

    def _score_canary(self, group: _Group) -> None:
        """δ̂ for every layer from the rows stashed on the fire step; the controllers
        take the fire before it."""
        rows, ctx = self.canary.stashed
        self.canary.stashed = None
        if self.canary.scored is not None:
            deltas, prev_ctx = self.canary.scored
            self.canary.scored = None
            for impl, d in zip(group.impls, deltas.tolist()):
                impl.controller.observe(dict(zip(SUPPORTED_BITS, d)), prev_ctx)
        planner = group.shared.planner
        if planner.kref_fill < self.cfg.k_group:
            return
        with record_function("echokv.canary"):
            kref = ring_view(torch.stack([i.kref_buf for i in group.impls]), planner.kref_pos, planner.kref_fill,
                             dim=1)
            q = torch.stack([i.stash[:rows] for i in group.impls])
            deltas = canary_kl(q, kref, SUPPORTED_BITS, self.cfg.k_group, group.impls[0].scale,
                               workspace=group.canary_ws)
            self.canary.scored = (_vllm.tp_mean(deltas), ctx)


# ---- implementation ----------------------------------------------------------------

class EchoKVAttentionImpl(AttentionImpl):
    # Decode workspaces shared by every layer of the process, by shape: layers run
    # one after another on one stream.
    _workspaces: ClassVar[dict] = {}

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int | None = None,
                 alibi_slopes: list[float] | None = None, sliding_window: int | None = None,
                 kv_cache_dtype: str = "auto", logits_soft_cap: float | None = None,
                 attn_type: str = AttentionType.DECODER, kv_sharing_target_layer_name: str | None = None,
                 sinks: torch.Tensor | None = None) -> None:
        unsupported = [name for name, bad in (
            ("alibi", alibi_slopes is not None),
            ("sliding window", sliding_window is not None),
            ("logits soft cap", bool(logits_soft_cap)),
            ("attention sinks", sinks is not None),
            ("KV sharing", kv_sharing_target_layer_name is not None),
            (f"attn_type={attn_type}", attn_type != AttentionType.DECODER),
        ) if bad]
        if unsupported:
            raise NotImplementedError(f"EchoKV does not support: {', '.join(unsupported)}")
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads or num_heads
        self.kv_cache_dtype = kv_cache_dtype
        self.cfg = cfg = load_config()
        if cfg.own_group_exact and not pf.own_group_takes(head_size, self.num_heads // self.num_kv_heads):
            raise NotImplementedError("ECHOKV_OWN_GROUP_EXACT needs head size 64 or 128 and GQA <= 128")
        self.controller = LayerController(cfg.controller)
        # Allocated at model construction so vLLM's memory profiler counts them: the
        # full-precision K of each block's open group (+1 spare row), the K_ref ring,
        # the canary's stashed query rows and the decode workspaces.
        dt = model_dtype()
        self.residual = torch.zeros(residual_slots(cfg) + 1, cfg.k_group, self.num_kv_heads, head_size, dtype=dt)
        self.kref_buf = torch.zeros(cfg.kref_window, self.num_kv_heads, head_size, dtype=torch.float32)
        self.stash = torch.zeros(cfg.canary_max_q, num_heads, head_size, dtype=dt)
        self._reserve_workspace(dt)
        self.store: TieredKVCache | None = None
        self.forward_calls = 0  # eager forwards; graph replays do not enter Python

    # -- buffers -------------------------------------------------------------------
    def _reserve_workspace(self, q_dtype: torch.dtype):
        """The decode workspace rows a graph-sized step needs, reserved now when a GPU is
        current (vLLM builds layers on the device) and shared by all layers."""
        vc = _vllm.current_vllm_config()
        if vc is None or not torch.cuda.is_available():
            return None
        cap = graph_capacity(vc)
        bs = getattr(getattr(vc, "cache_config", None), "block_size", None) or block_multiple()
        splits = decode_splits(vc.model_config.max_model_len, bs)
        layout = TieredLayout(self.num_kv_heads, self.head_size, bs, self.cfg.mem_bits, self.cfg.k_group,
                              self.cfg.v_group)
        from echokv_amd import _lib

        flags = _lib.DECODE_BATCH_INVARIANT if self.cfg.batch_invariant else 0
        rows = _lib.lib().echokv_decode_workspace_rows(_lib.byref(layout.abi(1, layout.page_bytes)), self.num_heads,
                                                       _lib.DTYPES[q_dtype], cap, splits, flags)
        if rows > 0:
            self._workspace(int(rows), torch.device("cuda", torch.cuda.current_device()))

    def _workspace(self, rows: int, device) -> tuple:
        """The process's shared workspace for this head shape, allocated once: a captured
        graph keeps its address, so it is never replaced by a larger one."""
        key = (str(device), self.num_heads, self.head_size)
        if key not in self._workspaces:
            self._workspaces[key] = (
                torch.empty(rows, self.num_heads, self.head_size, dtype=torch.float32, device=device),
                torch.empty(rows, self.num_heads, 2, dtype=torch.float32, device=device))
        return self._workspaces[key]

    def decode_workspace(self, n_dec: int, num_splits: int, cap: int) -> tuple | None:
        """``(acc, ml)`` for a decode of ``n_dec`` entries, or None (an eager step larger
        than any graph: the call allocates its own)."""
        store = self.store
        flags = 1 if self.cfg.batch_invariant else 0
        rows = dec.workspace_rows(store, self.num_heads, self.stash.dtype, n_dec, num_splits, flags)
        full = dec.workspace_rows(store, self.num_heads, self.stash.dtype, max(cap, n_dec), num_splits, flags)
        acc, ml = self._workspace(full, store.device)  # sized for the graph capacity on first use
        return (acc, ml) if acc.shape[0] >= rows else None

    def split_workspace(self, ws: tuple | None, n_dec: int, num_splits: int) -> tuple | None:
        """``ws`` if it holds the rows a split-schedule decode of ``n_dec`` entries needs,
        else None (the call allocates its own: eager steps only)."""
        rows = dec.workspace_rows(self.store, self.num_heads, self.stash.dtype, n_dec, num_splits, 1)
        return ws if ws is not None and ws[0].shape[0] >= rows else None

    def decode_tier(self) -> int:
        """The tier whose specialised decode kernel runs: the layer's current tier."""
        return self.controller.bits

    def bind(self, kv_cache: torch.Tensor, shared: SharedState) -> None:
        """Wrap ``kv_cache`` (this layer's view of vLLM's pool, ``[blocks, 1, block, bytes]``)."""
        raw = kv_cache.view(torch.uint8)
        shape = tuple(raw.shape)
        if raw.dim() != 4 or shape[1] != 1 or raw.stride(3) != 1 or raw.stride(2) != shape[3]:
            raise RuntimeError(f"unexpected EchoKV cache view shape={shape} stride={raw.stride()}")
        num_blocks, _, block_size, row = shape
        pages = raw.as_strided((num_blocks, block_size * row), (raw.stride(0), 1))
        layout = TieredLayout(self.num_kv_heads, self.head_size, block_size, self.cfg.mem_bits, self.cfg.k_group,
                              self.cfg.v_group)
        dev = pages.device
        self.residual, self.kref_buf, self.stash = (t.to(dev) for t in (self.residual, self.kref_buf, self.stash))
        self.store = TieredKVCache(layout, pages, residual=self.residual, shared=shared)

    # -- per layer and step -------------------------------------------------------
    @staticmethod
    def _step_metadata(layer):
        """This layer's metadata of the step (vLLM's forward context or a driver's)."""
        md = _vllm.forward_metadata()
        if isinstance(md, list):  # speculative decoding: the base model's metadata comes first
            md = md[0]
        if isinstance(md, dict):
            md = md[layer.layer_name]
        return md

    def do_kv_cache_update(self, layer, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                           slot_mapping: torch.Tensor) -> None:
        md = self._step_metadata(layer)
        if md is None or md.write is None:
            return
        with record_function("echokv.write"):
            self.store.apply(md.write, key, value, self.kref_buf, capturing=_capturing(key))

    def forward(self, layer, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                attn_metadata: EchoKVMetadata, output: torch.Tensor, output_scale: torch.Tensor | None = None,
                output_block_scale: torch.Tensor | None = None) -> torch.Tensor:
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("fused output quantization is not supported by EchoKV")
        md = attn_metadata
        if md is None or md.write is None:  # memory profiling / warm-up
            return output
        self.forward_calls += 1
        out = output.view(output.shape[0], -1, query.shape[-1])
        if md.prefill is not None:
            with record_function("echokv.prefill_attn"):
                md.prefill.run(self, query, key, md.block_table, out)
        if md.decode is not None:
            with record_function("echokv.decode_attn"):
                md.decode.run(self, query, md.block_table, out)
        # Stash the canary's query rows (scored at the next build); a graph records the
        # copy on every step, its rows being valid either way.
        if md.fire or _capturing(query):
            torch.index_select(query, 0, md.canary_rows, out=self.stash)
        return output


def _capturing(t: torch.Tensor) -> bool:
    return t.is_cuda and torch.cuda.is_current_stream_capturing()


def decode_splits(max_model_len: int, block_size: int) -> int:
    """The split grid of a decode: enough splits of ``BLOCKS_PER_SPLIT`` blocks for the
    longest sequence, at most ``MAX_DECODE_SPLITS``."""
    max_blocks = -(-max_model_len // block_size)
    return max(1, min(-(-max_blocks // dec.BLOCKS_PER_SPLIT), MAX_DECODE_SPLITS))


def graph_capacity(vllm_config) -> int:
    """The largest batch a captured graph replays (vLLM's capture sizes), 512 by default."""
    comp = getattr(vllm_config, "compilation_config", None)
    return getattr(comp, "max_cudagraph_capture_size", None) or 512


def residual_slots(cfg, vllm_config=None) -> int:
    """ECHOKV_RESIDUAL_SLOTS, else the scheduler's max_num_seqs + 16 (256 + 16 without one)."""
    if cfg.residual_slots is not None:
        return cfg.residual_slots
    vc = vllm_config if vllm_config is not None else _vllm.current_vllm_config()
    sched = getattr(vc, "scheduler_config", None)
    return (getattr(sched, "max_num_seqs", None) or 256) + 16


def model_dtype() -> torch.dtype:
    vc = _vllm.current_vllm_config()
    return vc.model_config.dtype if vc is not None else torch.float32
