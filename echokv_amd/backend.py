"""vLLM attention backend ("CUSTOM") over the MI355X tiered KV store.

Interface of ``echokv_vllm/backend.py:72-636``: ``EchoKVAttentionBackend``
(``customize_spec``, block / head-size support, ``get_name() == "CUSTOM"``),
``EchoKVMetadataBuilder`` (``build`` once per step for all layers) and
``EchoKVAttentionImpl`` (``bind``, ``do_kv_cache_update``, ``forward``). vLLM
budgets the page as one opaque byte state per token (``customize_spec``), so
its cache manager, memory profiler and block tables see exactly the bytes the
tiered store uses.

Per step the builder, on the host and once for every layer:

* plans the writes (native planner), seals evicted groups and opens blocks at
  each layer's current tier, and uploads the step's metadata with one
  non-blocking copy into a device image whose graph-visible parts sit at fixed
  offsets, so a captured decode graph reads each step's values;
* lays out the batch: one decode entry per single-token request (graph padding
  included, length 0), the prefill chunks with their work lists and one shared
  workspace;
* runs the canary for every layer at once on the step after a fire (δ̂ for every
  tier), and lets each layer's controller consume the previous fire's result, so
  reading it never waits for the stream.

``do_kv_cache_update`` and ``forward`` then only launch HIP kernels on device
metadata: the quantize-on-write of the step's K/V, chunked-prefill and decode
attention over the tiered pages (each block read at its own tier), and the copy
of the canary's query rows. There is no other path: without the HIP library the
calls raise.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, replace
from typing import ClassVar

import numpy as np
import torch

from echokv_amd import _vllm
from echokv_amd._util import to_device
from echokv_amd._vllm import (
    AttentionBackend,
    AttentionCGSupport,
    AttentionImpl,
    AttentionMetadataBuilder,
    AttentionType,
    MultipleOf,
)
from echokv_amd.canary import canary_kl, ring_view
from echokv_amd.config import load_config
from echokv_amd.controller import SUPPORTED_BITS, LayerController
from echokv_amd.host_slots import host_lens_and_slots, is_dummy_step
from echokv_amd.kernels import decode as dec
from echokv_amd.kernels import prefill as pf
from echokv_amd.tiered_cache import HeaderWriter, TieredKVCache, TieredLayout
from echokv_amd.write_plan import SharedState, WriteMeta

# Head sizes the MFMA kernels are built for; others up to MAX_HEAD_SIZE take the
# fp32 decode kernel (prefill through decode rows).
KERNEL_HEAD_SIZES = (64, 128)
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
        return head_size % 4 == 0 and head_size % load_config().v_group == 0 and head_size <= MAX_HEAD_SIZE

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


@dataclass
class EchoKVMetadata:
    num_actual_tokens: int
    num_reqs: int
    query_start_loc_cpu: torch.Tensor
    seq_lens_cpu: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    write: WriteMeta | None  # None: no KV cache bound yet (memory profiling); attention is skipped
    canary_rows: torch.Tensor | None  # [canary_max_q] query rows the canary reads
    fire: bool  # this step's query rows feed the canary (scored at the next build)
    decode_rows: torch.Tensor | None  # [nd] query rows of single-token requests
    decode_reqs: torch.Tensor | None  # [nd] their block-table rows
    decode_lens: torch.Tensor | None  # [nd] their cache lengths (0 = graph padding)
    num_splits: int  # decode split grid (fixed, so graphs can replay it)
    decode_workspace: tuple | None  # (acc, ml) shared by every layer's decode
    prefill: list  # (q_start, q_end, ctx, 0) per prefill request
    prefill_reqs: list  # block-table row of each prefill entry
    prefill_tiles: torch.Tensor | None  # fused-kernel tiles (every chunk <= 64 tokens)
    prefill_dense: object | None  # (DensePlan, workspace) of the two-pass path (longer chunks)
    own_group_rows: torch.Tensor | None = None  # own-group-exact prefill rows (ECHOKV_OWN_GROUP_EXACT=1)


class StepImage:
    """One step's int64 metadata in one device buffer, uploaded with one copy.

    Segments at fixed offsets (capacity ``cap`` rows, so a graph captured at any
    batch size up to ``cap`` reads the current step): ``[fin count | canary rows
    (nq) | decode q rows, block-table rows, lengths (3 x cap) | tokens (4 x cap) |
    fin rows (cap x w) | tail]``; the tail (residual map, page headers) is read by
    the builder's own index writes, never by a graph. A larger step uses a fresh
    buffer of its own size. Host images are pinned and reused round-robin once the
    copy that read them has completed.
    """

    RING = 4

    def __init__(self, cap: int, nq: int, w: int, tail: int, device) -> None:
        self.cap, self.nq, self.w, self.tail = cap, nq, w, tail
        self.device = torch.device(device)
        self.o_can = 2
        self.o_dec = self.o_can + nq + (nq & 1)
        self.o_tok = self.o_dec + 3 * cap
        self.o_fin = self.o_tok + 4 * cap
        self.o_tail = self.o_fin + cap * w
        self.size = self.o_tail + tail
        self.dev = torch.zeros(self.size, dtype=torch.long, device=self.device)
        pin = self.device.type == "cuda"
        self.host = [torch.zeros(self.size, dtype=torch.long, pin_memory=pin) for _ in range(self.RING if pin else 1)]
        self.done: list = [None] * len(self.host)
        self.turn = 0

    def upload(self, n_fin: int, canary: np.ndarray, decode: tuple, tok: np.ndarray, fin: np.ndarray, tail: list):
        """Views ``(fin_count, canary, (rows, reqs, lens), tok [4, t], fin, tail views)``."""
        nd, t = decode[0].size, tok.shape[1]
        tail_len = sum(a.size for a in tail)
        fits = max(nd, t, n_fin) <= self.cap and tail_len <= self.tail
        if fits:
            cap, o_dec, o_tok, o_fin, o_tail = self.cap, self.o_dec, self.o_tok, self.o_fin, self.o_tail
            fin_rows = cap  # a graph's finalize runs a full grid masked by the count
            i = self.turn
            if self.done[i] is not None:
                self.done[i].synchronize()  # the copy that read this host image four steps ago
            h = self.host[i].numpy()
        else:  # a step too large for any graph: a buffer of its own size
            cap = max(nd, t, n_fin, 1)
            o_dec = self.o_dec
            o_tok = o_dec + 3 * cap
            o_fin = o_tok + 4 * cap
            o_tail = o_fin + n_fin * self.w
            fin_rows = n_fin
            h = np.zeros(o_tail + tail_len, np.int64)
        h[0] = n_fin
        h[self.o_can : self.o_can + self.nq] = canary
        for k in range(3):
            h[o_dec + k * cap : o_dec + k * cap + nd] = decode[k]
        for k in range(4):
            h[o_tok + k * cap : o_tok + k * cap + t] = tok[k]
        h[o_fin : o_fin + fin.size] = fin.reshape(-1)
        o = o_tail
        for a in tail:
            h[o : o + a.size] = a.reshape(-1)
            o += a.size
        if fits:
            dev = self.dev
            dev[:o].copy_(self.host[i][:o], non_blocking=True)
            if self.device.type == "cuda":
                ev = self.done[i] or torch.cuda.Event()
                ev.record()
                self.done[i] = ev
            self.turn = (self.turn + 1) % len(self.host)
        else:
            dev = to_device(torch.from_numpy(h), self.device)
        views, o = [], o_tail
        for a in tail:
            views.append(dev[o : o + a.size])
            o += a.size
        return (dev[0:1], dev[self.o_can : self.o_can + self.nq],
                tuple(dev[o_dec + k * cap : o_dec + k * cap + nd] for k in range(3)),
                dev[o_tok : o_tok + 4 * cap].view(4, cap)[:, :t],
                dev[o_fin : o_fin + fin_rows * self.w].view(fin_rows, self.w), views)


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
        self.num_heads = _vllm.num_attention_heads(vllm_config, layer_names)
        self.gqa = self.num_heads // kv_cache_spec.num_kv_heads
        # Exact host sequence lengths are not available under async speculative decoding.
        self.host_slots = getattr(vllm_config, "speculative_config", None) is None
        self.check_host_slots = os.environ.get("ECHOKV_CHECK_HOST_SLOTS", "0") == "1"
        self.host_slot_steps = 0
        bs = kv_cache_spec.block_size
        max_blocks = -(-vllm_config.model_config.max_model_len // bs)
        self.num_splits = max(1, min(-(-max_blocks // dec.BLOCKS_PER_SPLIT), MAX_DECODE_SPLITS))
        self.residual_slots = residual_slots(self.cfg, vllm_config)
        comp = getattr(vllm_config, "compilation_config", None)
        self.cap = getattr(comp, "max_cudagraph_capture_size", None) or 512
        self.layers: list | None = None  # set by _attach (vLLM) or bind_layers (standalone)
        self.impls: list = []
        self._cache_ptr: int | None = None
        self.shared: SharedState | None = None
        self.image: StepImage | None = None
        self.workspace: tuple | None = None
        self.step = 0
        self.fire_pending = False
        self.measured: tuple | None = None  # (rows, mean context) stashed at the last fire
        self.pending: tuple | None = None  # the last δ̂ [layers, tiers] (device), not yet consumed

    # -- binding ----------------------------------------------------------------
    def bind_layers(self, layers: list) -> None:
        """The attention layers of this group (objects with ``kv_cache`` and ``impl``)."""
        self.layers = list(layers)
        self._cache_ptr = None

    def _attach(self) -> bool:
        """Bind every layer's impl to its KV cache and the shared state (once per cache)."""
        if self.layers is None:
            self.layers = _vllm.attention_layers(self.vllm_config, self.layer_names)
        first = getattr(self.layers[0], "kv_cache", None) if self.layers else None
        if first is not None and self._cache_ptr is not None and first.data_ptr() == self._cache_ptr:
            return True
        caches = [getattr(layer, "kv_cache", None) for layer in self.layers]
        if not caches or any(c is None or c.numel() == 0 for c in caches):
            return False  # memory profiling: no KV cache yet
        cfg = self.cfg
        self.shared = SharedState(caches[0].shape[0], self.kv_cache_spec.block_size, cfg.k_group, self.residual_slots,
                                  cfg.kref_window, self.device)
        self.impls = [layer.impl for layer in self.layers]
        for impl, cache in zip(self.impls, caches):
            impl.bind(cache, self.shared)
        self.headers = HeaderWriter([impl.store for impl in self.impls])
        tail = self.cap * (5 + 2 * len(self.impls)) + 64
        self.image = StepImage(self.cap, cfg.canary_max_q, 3 + cfg.k_group, tail, self.device)
        impl0 = self.impls[0]
        dev = torch.device(self.device)
        self.workspace = (torch.empty(self.cap, impl0.num_heads, self.num_splits, impl0.head_size, device=dev),
                          torch.empty(self.cap, impl0.num_heads, self.num_splits, 2, device=dev))
        self.canary_ws = torch.empty(len(self.impls) * impl0.num_kv_heads * len(SUPPORTED_BITS), device=dev)
        self._cache_ptr = caches[0].data_ptr()
        self.measured = self.pending = None
        return True

    # -- canary -----------------------------------------------------------------
    def _run_canary(self) -> None:
        """δ̂ for every layer from the query rows stashed on the fire step; the
        controllers consume the previous fire's δ̂ (long finished on the GPU)."""
        nq, ctx_mean = self.measured
        self.measured = None
        if self.pending is not None:
            deltas, prev_ctx = self.pending
            self.pending = None
            for impl, d in zip(self.impls, deltas.tolist()):
                impl.controller.observe(dict(zip(SUPPORTED_BITS, d)), prev_ctx)
        pl = self.shared.planner
        if pl.kref_fill < self.cfg.k_group:
            return
        kref = ring_view(torch.stack([i.kref_buf for i in self.impls]), pl.kref_pos, pl.kref_fill, dim=1)
        q = torch.stack([i.stash[:nq] for i in self.impls])
        deltas = canary_kl(q, kref, SUPPORTED_BITS, self.cfg.k_group, self.impls[0].scale, workspace=self.canary_ws)
        self.pending = (_vllm.tp_mean(deltas), ctx_mean)

    # -- build ------------------------------------------------------------------
    def build(self, common_prefix_len: int, common_attn_metadata, fast_build: bool = False) -> EchoKVMetadata:
        cm = common_attn_metadata
        if getattr(cm, "causal", True) is not True:
            raise NotImplementedError("EchoKV supports causal decoder attention only")
        n, t = cm.num_reqs, cm.num_actual_tokens
        bs = self.kv_cache_spec.block_size
        dummy = is_dummy_step(cm)
        host = host_lens_and_slots(cm, bs) if self.host_slots else None
        if host is not None:
            lens_cpu, slots_cpu = host
            self.host_slot_steps += 1
        if host is None and self.check_host_slots and self.host_slots and not dummy:
            raise AssertionError("ECHOKV_CHECK_HOST_SLOTS=1 but the host slot mapping is unavailable")
        if host is None or self.check_host_slots:
            # Device-to-host copies wait for the stream: only dummy steps and checks take them.
            dev_lens, dev_slots = cm.seq_lens[:n].cpu().long(), cm.slot_mapping[:t].cpu().long()
            if host is not None and not (torch.equal(lens_cpu, dev_lens) and torch.equal(slots_cpu, dev_slots)):
                raise AssertionError("EchoKV host slot mapping differs from vLLM's")
            lens_cpu, slots_cpu = dev_lens, dev_slots

        # The batch, vectorized over requests.
        qsl = cm.query_start_loc_cpu[: n + 1].numpy().astype(np.int64)
        lens = lens_cpu.numpy().astype(np.int64)
        qlen = np.diff(qsl)
        live = (qlen > 0) & (lens > 0)
        last_rows, last_ctx = (qsl[1:] - 1)[live], lens[live]
        if (qlen <= 1).all():
            d_idx = np.arange(n)  # decode-only, as graphs replay it: padding requests too (length 0)
        else:
            d_idx = np.flatnonzero(live & (qlen == 1))
        d_lens = np.where(qlen[d_idx] == 1, lens[d_idx], 0)
        d_rows = np.minimum(qsl[:-1][d_idx], max(t - 1, 0))
        pre = np.flatnonzero(live & (qlen > 1))
        prefill = [(int(qsl[r]), int(qsl[r + 1]), int(lens[r]), 0) for r in pre.tolist()]
        prefill_reqs = pre.tolist()

        write = canary_rows = None
        fire = False
        dec_views = (None, None, None)
        if self._attach():
            if self.measured is not None:
                self._run_canary()  # before this step's plan moves the K_ref ring
            if not dummy:
                self.step += 1
                if self.step % self.cfg.canary_interval == 0:
                    self.fire_pending = True
            nq = self.cfg.canary_max_q
            canary = np.zeros(nq, np.int64)
            if self.fire_pending and last_rows.size:
                self.fire_pending = False
                fire = True
                k = min(nq, last_rows.size)
                canary[:k] = last_rows[:k]
                self.measured = (k, float(last_ctx[:k].mean()))
            write, canary_rows, dec_views = self._plan(slots_cpu, canary, (d_rows, d_idx, d_lens))

        dev = self.device
        prefill_tiles = prefill_dense = None
        if prefill and self.impls and pf.kernels_take(self.impls[0].head_size, self.gqa):
            if not pf.use_dense(prefill, self.impls[0].head_size):
                prefill_tiles = pf.build_tiles(prefill, prefill_reqs, self.gqa, dev)
            else:
                plan = pf.build_dense_plan(prefill, prefill_reqs, self.gqa, dev)
                nbytes = pf.dense_workspace_bytes(self.impls[0].store, plan.packs.shape[0])
                prefill_dense = (plan, torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev))
        og_rows = pf.build_own_group_rows(prefill, prefill_reqs, dev) if prefill and self.cfg.own_group_exact else None
        return EchoKVMetadata(
            num_actual_tokens=t, num_reqs=n, query_start_loc_cpu=cm.query_start_loc_cpu[: n + 1].cpu(),
            seq_lens_cpu=lens_cpu, block_table=cm.block_table_tensor, slot_mapping=cm.slot_mapping, write=write,
            canary_rows=canary_rows, fire=fire, decode_rows=dec_views[0] if d_idx.size else None,
            decode_reqs=dec_views[1] if d_idx.size else None, decode_lens=dec_views[2] if d_idx.size else None,
            num_splits=self.num_splits,
            decode_workspace=self.workspace if d_idx.size and d_idx.size <= self.cap else None,
            prefill=prefill, prefill_reqs=prefill_reqs, prefill_tiles=prefill_tiles, prefill_dense=prefill_dense,
            own_group_rows=og_rows)

    def _plan(self, slots_cpu: torch.Tensor, canary: np.ndarray, decode: tuple):
        """Host side of the step's writes for every layer, then one upload."""
        shared = self.shared
        plan = shared.planner.plan(slots_cpu)
        # Which blocks open is the same in every layer (offset-0 writes and writes into
        # never-opened blocks); the tier each opens at is the layer's own.
        opens = self.impls[0].store.pool.fresh_opens(plan)
        opened = []
        if opens.size or plan.evictions:
            for impl in self.impls:
                st = impl.store
                for ev in plan.evictions:  # rare; before the slot is reused below
                    st._seal(ev)
                if opens.size:
                    opened.append(st.open_blocks(opens, impl.controller.bits, protect=plan.touched_np))
        shared.commit(plan)
        tail = [plan.res_map_block, plan.res_map_value, plan.res_group_slot, plan.res_group_value]
        if opened:  # the same blocks in every layer: their ids once, then each layer's headers
            self.headers.check(opens)
            tail += [opens, np.concatenate([np.ascontiguousarray(h).view(np.int64).reshape(-1) for _, h in opened])]
        tok = np.stack([plan.tok_slot, plan.tok_res, plan.tok_sealed, plan.tok_kref])
        fin_count, canary_rows, dec_views, tok_d, fin_d, views = self.image.upload(
            plan.n_fin, canary, decode, tok, plan.fin, tail)
        shared.apply_res_map(*views[:4])
        if opened:
            self.headers.write(views[4], views[5])
        write = WriteMeta(tok=tok_d, fin=fin_d, fin_count=fin_count, n_rows=plan.n_rows, n_fin=plan.n_fin)
        return write, canary_rows, dec_views


class EchoKVAttentionImpl(AttentionImpl):
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
        if cfg.own_group_exact and not pf.kernels_take(head_size, self.num_heads // self.num_kv_heads):
            raise NotImplementedError("ECHOKV_OWN_GROUP_EXACT needs head size 64 or 128 and GQA <= 128")
        self.controller = LayerController(cfg.controller)
        # Allocated at model construction so vLLM's memory profiler counts them: the
        # full-precision K of each block's open group (+1 spare row), the K_ref ring and
        # the canary's stashed query rows.
        dt = model_dtype()
        self.residual = torch.zeros(residual_slots(cfg) + 1, cfg.k_group, self.num_kv_heads, head_size, dtype=dt)
        self.kref_buf = torch.zeros(cfg.kref_window, self.num_kv_heads, head_size, dtype=torch.float32)
        self.stash = torch.zeros(cfg.canary_max_q, num_heads, head_size, dtype=dt)
        self.store: TieredKVCache | None = None
        self.forward_calls = 0  # eager forwards; graph replays do not enter Python

    def bind(self, kv_cache: torch.Tensor, shared: SharedState) -> None:
        """Wrap ``kv_cache`` (this layer's view of vLLM's pool, ``[blocks, 1, block, bytes]``)."""
        raw = kv_cache.view(torch.uint8)
        if raw.dim() != 4:
            raise RuntimeError(f"unexpected EchoKV cache view shape={tuple(raw.shape)}")
        num_blocks, slots, block_size, row = raw.shape
        if slots != 1 or raw.stride(3) != 1 or raw.stride(2) != row:
            raise RuntimeError(f"unexpected EchoKV cache view shape={tuple(raw.shape)} stride={raw.stride()}")
        pages = torch.as_strided(raw, (num_blocks, block_size * row), (raw.stride(0), 1))
        layout = TieredLayout(self.num_kv_heads, self.head_size, block_size, self.cfg.mem_bits, self.cfg.k_group,
                              self.cfg.v_group)
        dev = pages.device
        self.residual = self.residual.to(dev)
        self.kref_buf = self.kref_buf.to(dev)
        self.stash = self.stash.to(dev)
        self.store = TieredKVCache(layout, pages, residual=self.residual, shared=shared)

    # -- write path --------------------------------------------------------------
    def do_kv_cache_update(self, layer, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                           slot_mapping: torch.Tensor) -> None:
        md = _vllm.forward_metadata()
        if isinstance(md, list):  # speculative decoding: [0] is the base model
            md = md[0]
        if isinstance(md, dict):
            md = md[layer.layer_name]
        if md is None or md.write is None:
            return
        self.store.apply(md.write, key, value, self.kref_buf, capturing=_capturing(key))

    # -- read path ---------------------------------------------------------------
    def forward(self, layer, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                attn_metadata: EchoKVMetadata, output: torch.Tensor, output_scale: torch.Tensor | None = None,
                output_block_scale: torch.Tensor | None = None) -> torch.Tensor:
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("fused output quantization is not supported by EchoKV")
        md = attn_metadata
        if md is None or md.write is None:  # profiling / warm-up run
            return output
        self.forward_calls += 1
        store = self.store
        out = output.view(output.shape[0], -1, query.shape[-1])
        if md.prefill:
            og_key = None
            if md.own_group_rows is not None:  # own-group-exact: this step's key rows, aligned with the queries
                og_key = key.view(key.shape[0], self.num_kv_heads, self.head_size)
            pf.prefill_attention(store, query, out, md.prefill, md.prefill_reqs, md.block_table, self.scale,
                                 tiles=md.prefill_tiles, dense=md.prefill_dense, own_group_key=og_key,
                                 own_group_rows=md.own_group_rows)
        if md.decode_rows is not None:
            # Query / block-table rows by index, output rows written in place.
            dec.decode_attention(store, query, md.block_table, md.decode_lens, self.scale, q_rows=md.decode_rows,
                                 bt_rows=md.decode_reqs, out=out, num_splits=md.num_splits,
                                 workspace=md.decode_workspace, tier=self.controller.bits)
        # The canary's query rows (scored at the next build). A graph captures the
        # copy unconditionally: its rows are valid either way.
        if md.fire or _capturing(query):
            torch.index_select(query, 0, md.canary_rows, out=self.stash)
        return output


def _capturing(t: torch.Tensor) -> bool:
    return t.is_cuda and torch.cuda.is_current_stream_capturing()


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
