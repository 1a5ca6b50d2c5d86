"""One engine step's host work for every layer of a KV-cache group, uploaded in one copy.

This replaces the reference builder's per-step host path (``_plan`` and
``_Staging``, ``echokv_vllm/backend.py:144-229,463-496``) with one native call
(``ekh_stepper_run``, ``echokv_amd/host/step.cpp``) that lays out the batch,
plans the writes, opens the step's blocks in every layer's pool at that layer's
tier and writes the whole result as one int64 image, straight into pinned host
memory. ``StepDriver.run`` then issues one host-to-device copy and returns
device views of each part.

The image's graph-visible parts (counts, canary rows, decode entries, token and
fin rows) sit at offsets fixed by the capacity in one persistent device buffer,
so a HIP graph captured at any batch size up to the capacity reads the current
step. A step larger than that (a long prefill) is never graph-replayed and gets
a device buffer of its own. Pinned host images rotate through a small ring; a
slot is rewritten only once the copy that read it has completed.
"""

from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass

import numpy as np
import torch

from echokv_amd import _host
from echokv_amd._util import to_device


@dataclass
class StepUpload:
    """A step's device views and the host facts the builder needs."""

    fin_count: torch.Tensor  # [1]: masks a graph's full-grid finalize
    canary_rows: torch.Tensor  # [canary slots] query rows the canary reads on a fire step
    tier_masks: torch.Tensor  # [layers, 2] int32: element [l, 0] holds layer l's live tiers (2 | 4 | 8)
    host_tier_masks: np.ndarray  # [layers] the same on the host
    decode: tuple | None  # (query rows, block-table rows, lengths), [n_dec] each; None: no decode entry
    tok: torch.Tensor  # [4, n_tokens] (row stride = capacity): slot, residual slot, sealed, K_ref row
    fin: torch.Tensor  # [fin rows, 3 + k_group]; the first n_fin are this step's
    res_map: tuple  # (blocks, values, residual slots, groups): residual-map updates
    open_ids: torch.Tensor  # [n_open] blocks opened this step
    headers: torch.Tensor  # [layers * n_open * 2] int64: their page headers, layer-major
    seal_rows: list  # per layer, [n_seal, 6] device rows sealing evicted groups (empty when none)
    victims: np.ndarray  # [n, 2] (layer, block): full blocks to requantize to INT2 before the headers
    prefill: list  # (q_start, q_end, context, request) per prefill entry
    n_tokens: int
    n_fin: int
    n_canary: int  # canary rows taken (0: no fire this step)
    canary_ctx: float


class StepDriver:
    """``ekh_stepper`` over a planner and its layers' pools, plus the upload ring.

    ``RING`` pinned images: the host plans step i + RING only once the copy of
    step i has run, so it stays at most ``RING`` steps ahead of the device. One is
    enough to keep a graph-replayed decode step fed (the next step is planned while
    the current one runs) and keeps the stream's queue short: with the host four
    steps ahead, the runtime now and then held a small pinned copy for 6-10 ms
    until its queue drained, and the device then waited on the host (32-layer cfg2
    step: 4.50 ms at four images, 4.35 at two, 4.18 at one, against 4.13 ms of
    kernels)."""

    RING = 1

    def __init__(self, shared, stores, cap: int, canary_slots: int, device) -> None:
        lib = _host.lib()
        self.n_layers = len(stores)
        pools = (C.c_void_p * self.n_layers)(*[s.pool._h.value for s in stores])
        h = lib.ekh_stepper_new(shared.planner._h, pools, self.n_layers, cap, canary_slots)
        if not h:
            raise ValueError("cannot drive these layers: every pool must share the group's planner")
        self._h = C.c_void_p(h)
        self._free_fn = lib.ekh_stepper_free
        self._keep = (shared, list(stores))  # the native planner and pools outlive the stepper
        self.cap = cap + cap % 2
        self.nq = canary_slots
        self.w = 3 + shared.planner.g
        self.device = torch.device(device)
        head = 2 + self.nq + self.nq % 2 + self.n_layers + self.n_layers % 2 + 7 * self.cap + self.cap * self.w
        tail = self.cap * (5 + 2 * self.n_layers) + 6 * self.n_layers * 8 + 64
        self.words = head + tail
        self.dev = torch.zeros(self.words, dtype=torch.int64, device=self.device)
        pin = self.device.type == "cuda"
        self.host = [torch.zeros(self.words, dtype=torch.int64, pin_memory=pin) for _ in range(self.RING if pin else 1)]
        self.copied: list = [None] * len(self.host)
        self.turn = 0
        self.wait_s = 0.0  # host time spent waiting for a ring slot (the host ran RING steps ahead)
        self._view = _host.StepView()

    def __del__(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._free_fn(h)
            self._h = None

    def run(self, qsl: np.ndarray, lens: np.ndarray, slots: np.ndarray, tiers: np.ndarray, fire: bool) -> StepUpload:
        """Plan and upload one step. ``qsl`` [n + 1] and ``lens`` [n] int32, ``slots``
        [t] int64 (-1: no write), ``tiers`` [layers] int32."""
        n, t = lens.size, slots.size
        batch = _host.Batch(n, t, qsl.ctypes.data, lens.ctypes.data, slots.ctypes.data)
        i = self.turn
        if self.copied[i] is not None:
            t_wait = time.perf_counter()
            self.copied[i].synchronize()  # the copy that read this image RING steps ago
            self.wait_s += time.perf_counter() - t_wait
        buf = self.host[i]
        v = self._view
        rc = _host.lib().ekh_stepper_run(self._h, C.byref(batch), tiers.ctypes.data, int(fire), buf.data_ptr(),
                                         self.words, C.byref(v))
        if rc == _host.ESLOTS:
            raise RuntimeError("more open K groups in one step than residual slots (ECHOKV_RESIDUAL_SLOTS)")
        if rc != _host.OK:
            raise ValueError("invalid step: query starts, lengths or slots outside the cache group")
        in_ring = C.cast(v.image, C.c_void_p).value == buf.data_ptr()
        if v.graph_rows:
            # The graph-visible head goes to the persistent buffer, always at the same address.
            if not in_ring:  # a tail too large for the ring's images: the head is copied in
                np.copyto(buf.numpy()[: v.o_res], np.ctypeslib.as_array(v.image, shape=(v.o_res,)))
            upto = v.len if in_ring else v.o_res
            self.dev[:upto].copy_(buf[:upto], non_blocking=True)
            if self.device.type == "cuda":
                ev = self.copied[i] or torch.cuda.Event()
                ev.record()
                self.copied[i] = ev
            self.turn = (i + 1) % len(self.host)
            head = self.dev
            tail = self.dev if in_ring else self._own(v.image, v.o_res, v.len)
            t0 = 0 if in_ring else v.o_res
        else:  # never graph-replayed: a device buffer of its own
            head = tail = self._own(v.image, 0, v.len)
            t0 = 0
        return self._views(v, head, tail, t0)

    def apply(self, up: StepUpload, headers) -> None:
        """The step's device effects the layers' writes depend on, in stream order:
        seal evicted groups, demote pool victims to INT2, then the residual-map and
        page-header updates (``headers``: the group's ``HeaderWriter``)."""
        shared, stores = self._keep
        for store, rows in zip(stores, up.seal_rows):
            store.seal_groups(rows)
        for layer in np.unique(up.victims[:, 0]).tolist():
            stores[layer]._demote(up.victims[up.victims[:, 0] == layer, 1].tolist())
        shared.apply_res_map(*up.res_map)
        if up.open_ids.numel():  # ids the planner checked against the pool
            headers.write(up.open_ids, up.headers)

    def _own(self, image, start: int, end: int) -> torch.Tensor:
        host = np.ctypeslib.as_array(image, shape=(end,))[start:end].copy()
        return to_device(torch.from_numpy(host), self.device)

    def _views(self, v, head: torch.Tensor, tail: torch.Tensor, t0: int) -> StepUpload:
        def seg(o, n):
            return tail[o - t0 : o - t0 + n]

        dec = None
        if v.n_dec:
            dec = tuple(head[v.o_dec + k * v.rows_dec : v.o_dec + k * v.rows_dec + v.n_dec] for k in range(3))
        seal = []
        if v.n_seal:
            rows = seg(v.o_seal, 6 * v.n_seal * self.n_layers).view(self.n_layers, v.n_seal, 6)
            seal = list(rows.unbind(0))
        prefill = []
        if v.n_prefill:
            prefill = [tuple(r) for r in np.ctypeslib.as_array(v.prefill, shape=(v.n_prefill, 4)).tolist()]
        victims = np.zeros((0, 2), np.int64)
        if v.n_victims:
            victims = np.ctypeslib.as_array(v.victims, shape=(v.n_victims, 2)).copy()
        return StepUpload(
            fin_count=head[0:1],
            canary_rows=head[v.o_canary : v.o_canary + self.nq],
            tier_masks=head[v.o_mask : v.o_mask + self.n_layers].view(torch.int32).view(self.n_layers, 2),
            host_tier_masks=np.ctypeslib.as_array(v.image, shape=(v.o_mask + self.n_layers,))[v.o_mask :].copy(),
            decode=dec,
            tok=head[v.o_tok : v.o_tok + 4 * v.rows_tok].view(4, v.rows_tok)[:, : v.n_tokens],
            fin=head[v.o_fin : v.o_fin + v.rows_fin * self.w].view(v.rows_fin, self.w),
            res_map=(seg(v.o_res, v.n_res), seg(v.o_res + v.n_res, v.n_res), seg(v.o_grp, v.n_grp),
                     seg(v.o_grp + v.n_grp, v.n_grp)),
            open_ids=seg(v.o_open, v.n_open),
            headers=seg(v.o_hdr, 2 * v.n_open * self.n_layers),
            seal_rows=seal, victims=victims, prefill=prefill, n_tokens=int(v.n_tokens), n_fin=int(v.n_fin),
            n_canary=int(v.n_canary), canary_ctx=float(v.canary_ctx))
