"""Benchmark: BASELINE config 2 -- Llama-3.1-8B-shaped paged decode over a mixed-tier
quantized KV cache on one MI355X.

32 layers, each Hq=32 / H=8 / D=128, page block 16, K group 16, V group 32,
mem_bits 8 pages; tier vector = a seeded permutation of 8 x INT8, 16 x INT4,
8 x INT2; batch 64 with context lengths ~U[512, 8192] (seed 1); fp16 K/V/Q
~N(0,1) with 1% of the K and of the V (head, channel) pairs x10 (outliers). One step = for
every layer, quantize-on-write of one new token per sequence (the fused write
step: finalize of the completing K groups and the token rows in one launch) then
decode attention (balanced schedule: decode + merge), all on the device; the host
plans the step's writes once for all layers.

Prints one JSON line. ``value`` = INT4 paged-decode attention throughput in
GB/s of algorithmic bytes (K/V codes, stats, residual, Q, O that the math
needs): the 16 INT4 layers' decode (decode + merge kernels, each layer over its
own pages, at the lengths the timed steps reached) captured as one HIP graph
and replayed ``--reps`` times between HIP events on the launch stream, so the
time is GPU work only; ``roofline`` puts it against 8 TB/s. ``ms_per_step`` and
``attn_write_step_tok_s`` time the whole 32-layer attention + KV-write step (host
planning included; no model: no projections, MLP or sampling) over the
``--steps`` timed steps, each replayed as one HIP graph (the plan staged into
fixed device buffers); ``attn_write_step_eager_*`` times the same steps launched
one kernel at a time. ``host_plan_us`` is the host's share of a step (plan,
chunk-pool opens, staging) at 64 sequences, and at 256 on the planner alone.
``hbm_copy_ceiling_GBs`` is the same run's 1 GiB device copy rate (read + write).

``cpu_baseline``: the reference's PyTorch path restated in torch on the host cores
(``oracle/torch_cpu.py``): decode of the whole INT4 layer-step, repeated to about
10 s (``value``, GB/s of the same algorithmic bytes), one step's writes, 512-token
prefill chunks and one canary fire of a layer.

``prefill`` (one layer): 16 sequences x 4096 tokens written
and attended in 512-token chunks over an INT4 cache, bf16 activations; per
chunk the quantize-on-write of its tokens, then chunked-prefill attention over
the whole context written so far (the two-pass path: workspace pack + flash
kernel), timed with HIP events; utilisation = 4 D Hq (causal pairs) / time
against 2.5 PFLOP/s dense fp16.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "INT4 paged-decode attn HBM GB/s (% of peak); e2e decode tok/s at 8B shape"
HBM_PEAK_GBS = 8000.0

H, HQ, D, BS, KG, VG, MEM, LAYERS, S = 8, 32, 128, 16, 16, 32, 8, 32, 64
PF_SEQS, PF_CTX, PF_CHUNK = 16, 4096, 512  # config 3
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16


def alg_bytes(lens: np.ndarray, bits: int, res_bytes: int = 2, hq: int = HQ) -> int:
    """Decode bytes of one layer-step: what the attention math must read / write."""
    g = D // VG
    sealed_grp = lens // KG
    open_tok = lens % KG
    sealed_tok = sealed_grp * KG
    per_sealed = 2 * H * D * bits // 8 + H * g * 4
    per_open = H * D * bits // 8 + H * g * 4 + H * D * res_bytes
    kv = sealed_tok * per_sealed + sealed_grp * H * D * 4 + open_tok * per_open
    return int(kv.sum()) + 2 * len(lens) * hq * D * 2


def build_state(dev, steps_total: int, seed: int = 1):
    import torch

    from echokv_amd.tiered_cache import TieredKVCache, TieredLayout
    from echokv_amd.write_plan import SharedState, stage_plan

    rng = np.random.default_rng(seed)
    ctx = rng.integers(512, 8193, S).astype(np.int64)
    tiers = rng.permutation(np.array([8] * 8 + [4] * 16 + [2] * 8))
    layout = TieredLayout(H, D, BS, MEM, KG, VG)
    page = layout.aligned_stride  # pages on 128-byte lines (see TieredLayout.alloc_pages)
    nbs = -(-(ctx + steps_total + 1) // BS)
    nb = int(nbs.sum()) + 16
    perm = rng.permutation(nb)
    table = np.zeros((S, int(nbs.max())), np.int64)
    o = 0
    for i, n in enumerate(nbs):
        table[i, :n] = perm[o : o + n]
        o += n
    shared = SharedState(nb, BS, KG, S + 16, kref_window=64, device=dev)
    stores, krefs = [], []
    for _ in range(LAYERS):
        pages = layout.alloc_pages(nb, dev)
        res = torch.zeros(S + 17, KG, H, D, dtype=torch.float16, device=dev)
        stores.append(TieredKVCache(layout, pages, residual=res, shared=shared))
        krefs.append(torch.zeros(64, H, D, device=dev))
    # Prefill every sequence's first ctx-1 tokens, all layers, one planned step.
    pre = np.concatenate([table[i][np.arange(n - 1) // BS] * BS + np.arange(n - 1) % BS for i, n in enumerate(ctx)])
    plan = shared.planner.plan(pre)
    opened = [st.prepare(plan, int(t)) for st, t in zip(stores, tiers)]
    shared.commit(plan)
    meta, extra = stage_plan(plan, dev, None)
    shared.apply_res_map(*extra[:4])
    gen = torch.Generator(device=dev)
    for li, (st, op) in enumerate(zip(stores, opened)):
        if op is not None:
            st.write_headers(torch.from_numpy(op[0]).to(dev), torch.from_numpy(op[1]).to(dev))
        gen.manual_seed(1000 + li)
        k = torch.randn(pre.size, H, D, device=dev, dtype=torch.float16, generator=gen)
        v = torch.randn(pre.size, H, D, device=dev, dtype=torch.float16, generator=gen)
        out_ch = torch.randperm(H * D, generator=gen, device=dev)[: round(0.01 * H * D)]
        k.view(pre.size, H * D)[:, out_ch] *= 10
        v_ch = torch.randperm(H * D, generator=gen, device=dev)[: round(0.01 * H * D)]
        v.view(pre.size, H * D)[:, v_ch] *= 10
        st.apply(meta, k, v, krefs[li])
        del k, v
    torch.cuda.synchronize()
    return dict(ctx=ctx, tiers=tiers, table=table, shared=shared, stores=stores, krefs=krefs, nb=nb, page=page)


def run(args) -> dict:
    import torch

    from echokv_amd.kernels.decode import decode_attention
    from echokv_amd.step import StepDriver
    from echokv_amd.tiered_cache import HeaderWriter
    from echokv_amd.write_plan import WriteMeta

    dev = torch.device("cuda:0")
    t_setup = time.time()
    host_steps = 20
    st = build_state(dev, args.warmup + 2 * args.steps + 2 + host_steps)
    ctx, tiers, table = st["ctx"], st["tiers"], st["table"]
    shared, stores, krefs = st["shared"], st["stores"], st["krefs"]
    print(f"[bench] state ready: {st['nb']} blocks/layer, {st['nb'] * st['page'] * LAYERS / 2**30:.1f} GiB pages, "
          f"{time.time() - t_setup:.1f}s", file=sys.stderr, flush=True)
    table_d = torch.from_numpy(table).to(dev, torch.int32)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    q = [torch.randn(S, HQ, D, device=dev, dtype=torch.float16, generator=gen) for _ in range(LAYERS)]
    kn = [torch.randn(S, H, D, device=dev, dtype=torch.float16, generator=gen) for _ in range(LAYERS)]
    vn = [torch.randn(S, H, D, device=dev, dtype=torch.float16, generator=gen) for _ in range(LAYERS)]
    out = [torch.empty(S, HQ, D, device=dev, dtype=torch.float16) for _ in range(LAYERS)]
    max_blocks = table.shape[1]
    num_splits = max(1, min(-(-max_blocks // args.bps), args.max_splits))
    ws = (torch.empty(S, HQ, num_splits, D, device=dev), torch.empty(S, HQ, num_splits, 2, device=dev))
    int4 = [li for li in range(LAYERS) if tiers[li] == 4]
    scale = D ** -0.5
    inv = args.schedule == "split"
    headers = HeaderWriter(stores)
    # The product's per-step host path: one native call plans the step for all 32
    # layers (write plan, opened blocks and headers per layer) into one image, one
    # copy uploads it, and the device effects are launched (StepDriver, as the
    # vLLM backend's builder runs it).
    driver = StepDriver(shared, stores, cap=S, canary_slots=8, device=dev)
    tiers32 = tiers.astype(np.int32)
    qsl = np.arange(S + 1, dtype=np.int32)

    def host_step(i):
        pos = ctx - 1 + i  # position of this step's new token
        slots = (table[np.arange(S), pos // BS] * BS + pos % BS).astype(np.int64)
        up = driver.run(qsl, (pos + 1).astype(np.int32), slots, tiers32, False)
        driver.apply(up, headers)
        return up, pos + 1

    def step(i):
        up, lens = host_step(i)
        meta = WriteMeta(tok=up.tok, fin=up.fin, fin_count=up.fin_count, n_rows=up.n_tokens, n_fin=up.n_fin)
        rows, reqs, lens_d = up.decode
        for li, s in enumerate(stores):
            s.apply(meta, kn[li], vn[li], krefs[li])
            decode_attention(s, q[li], table_d, lens_d, scale, blocks_per_split=args.bps, q_rows=rows, bt_rows=reqs,
                             out=out[li], num_splits=num_splits, workspace=ws, tier=int(tiers[li]),
                             batch_invariant=inv)
        return lens

    # End to end, eager: the host plans every step; all 32 layers write and attend.
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + args.steps):
        lens = step(i)
    torch.cuda.synchronize()
    wall_eager = time.perf_counter() - t0

    # End to end, graph-replayed (as a serving engine runs decode): the host plans
    # each step into the driver's fixed device buffers (rows = the batch, finalize
    # over a full grid masked by the device count); one HIP graph then runs every
    # layer's finalize, write, decode and merge.
    g0 = args.warmup + args.steps
    up, lens = host_step(g0)
    gmeta = WriteMeta(tok=up.tok, fin=up.fin, fin_count=up.fin_count, n_rows=S, n_fin=up.fin.shape[0])
    g_rows, g_reqs, g_lens = up.decode

    def all_layers():
        for li, s in enumerate(stores):
            s.apply(gmeta, kn[li], vn[li], krefs[li], capturing=True)
            decode_attention(s, q[li], table_d, g_lens, scale, blocks_per_split=args.bps, q_rows=g_rows,
                             bt_rows=g_reqs, out=out[li], num_splits=num_splits, workspace=ws, tier=int(tiers[li]),
                             batch_invariant=inv)

    all_layers()  # step g0, eagerly (its plan is staged)
    torch.cuda.synchronize()
    step_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(step_graph):
        all_layers()

    host_s = [0.0]

    def gstep(i):
        t_host = time.perf_counter()
        up, lens = host_step(i)
        assert up.tok.data_ptr() == gmeta.tok.data_ptr() and up.decode[2].data_ptr() == g_lens.data_ptr()
        host_s[0] += time.perf_counter() - t_host
        step_graph.replay()
        return lens

    for i in range(g0 + 1, g0 + 2):
        gstep(i)
    torch.cuda.synchronize()
    host_s[0] = 0.0
    driver.wait_s = 0.0
    t0 = time.perf_counter()
    for i in range(g0 + 2, g0 + 2 + args.steps):
        lens = gstep(i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    host_s[0] -= driver.wait_s  # the host ran ahead of the GPU: waits for a ring slot are not host work
    # The host's share of a step alone: steps taken with the GPU drained first, so
    # launch back-pressure from queued graph replays is not counted -- the native
    # stepper, the upload and the launches of the step's device effects.
    g1 = g0 + 2 + args.steps
    host_times = []
    for i in range(g1, g1 + host_steps):
        torch.cuda.synchronize()
        t_host = time.perf_counter()
        up, lens = host_step(i)
        host_times.append(time.perf_counter() - t_host)
        step_graph.replay()
    torch.cuda.synchronize()

    # The metric: the 16 INT4 layers' decode attention (decode + merge kernels) over
    # their own pages, at the lengths the last step reached, replayed as one HIP
    # graph so the events time GPU work only (no host launch gaps).
    lens_d = torch.from_numpy(lens).to(dev)

    def time_int4(invariant: bool) -> float:
        """ms per INT4 layer-step (decode + merge), graph-replayed over the 16 INT4 layers."""
        def int4_decode():
            for li in int4:
                decode_attention(stores[li], q[li], table_d, lens_d, scale, blocks_per_split=args.bps, out=out[li],
                                 num_splits=num_splits, workspace=ws, tier=4, batch_invariant=invariant)

        int4_decode()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            int4_decode()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (len(int4) * args.reps)

    avg_ms = time_int4(inv)
    other_ms = time_int4(not inv)
    per_layer_bytes = alg_bytes(lens, 4)
    achieved = per_layer_bytes / (avg_ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8 codes (INT4) -> fp16 MFMA, fp32 accumulate",
        "data": "synthetic: fp16 K/V/Q ~N(0,1), 1% of K and of V channels x10; random block tables",
        "config": {
            "workload": "cfg2: Llama-3.1-8B-shaped decode, 32 layers (8 INT8 / 16 INT4 / 8 INT2), batch 64, "
                        "ctx ~U[512,8192], Hq 32 / H 8 / D 128, page block 16, K group 16, V group 32",
            "global_batch": S,
            "seq_len": int(ctx.mean()),
            "parallelism": "single GPU",
        },
        "attn_write_step_tok_s": round(S * args.steps / wall, 1),
        "host_plan_us": {"64": round(float(np.median(host_times)) * 1e6, 1),
                         "64, in the replay loop": round(host_s[0] / args.steps * 1e6, 1),
                         "256 (planner only)": plan_only_us(256)},
        "attn_write_step_eager_ms": round(wall_eager * 1e3 / args.steps, 3),
        "attn_write_step_eager_tok_s": round(S * args.steps / wall_eager, 1),
        "int4_decode_us_per_layer": round(avg_ms * 1e3, 2),
        "schedule": args.schedule,
        "other_schedule": {"schedule": "split" if not inv else "balanced",
                           "int4_decode_us_per_layer": round(other_ms * 1e3, 2),
                           "GBs": round(alg_bytes(lens, 4) / (other_ms * 1e-3) / 1e9, 1)},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "kernel": ("decode_kernel<128, 4> + merge_kernel" if inv else "decode_balanced_kernel<128, 4> + merge_balanced_kernel")
                      + " (one INT4 layer-step, graph replay over the 16 INT4 layers)",
            "alg_bytes_per_launch": int(per_layer_bytes),
        },
    }
    res["hbm_copy_ceiling_GBs"] = copy_ceiling(dev)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(stores[int4[0]], shared, q[int4[0]], kn[int4[0]], vn[int4[0]], table, lens)
    if not args.no_prefill:
        res["prefill"] = run_prefill()
    if not args.no_mixed:
        res["mixed_tier"] = run_mixed()
        res["head_size_256"] = run_d256()
    return res


def prefill_flops(ctx: int, chunk: int, seqs: int) -> int:
    """QK^T + PV flops of one chunk: 4 D Hq per (query, visible key) pair, causal."""
    pairs = seqs * (chunk * (ctx - chunk) + chunk * (chunk + 1) // 2)
    return 4 * D * HQ * pairs


def run_prefill(reps: int = 3) -> dict:
    """Config 3 on one layer: every 512-token chunk of 16 x 4096 tokens is written
    (quantize-on-write into INT4 pages) and attended over its whole context. A
    first pass over a fresh cache warms every kernel up; the second is timed."""
    _prefill_pass(1)
    return _prefill_pass(reps)


def _prefill_pass(reps: int) -> dict:
    import torch

    from echokv_amd.kernels import prefill as pf
    from echokv_amd.tiered_cache import TieredKVCache, TieredLayout
    from echokv_amd.write_plan import SharedState, stage_plan

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(3)
    layout = TieredLayout(H, D, BS, MEM, KG, VG)
    page = layout.aligned_stride  # pages on 128-byte lines (see TieredLayout.alloc_pages)
    nbs = PF_CTX // BS
    nb = PF_SEQS * nbs + 16
    table = rng.permutation(nb)[: PF_SEQS * nbs].reshape(PF_SEQS, nbs).astype(np.int64)
    shared = SharedState(nb, BS, KG, PF_SEQS + 16, kref_window=64, device=dev)
    pages = layout.alloc_pages(nb, dev, zero=True)
    res = torch.zeros(PF_SEQS + 17, KG, H, D, dtype=torch.bfloat16, device=dev)
    store = TieredKVCache(layout, pages, residual=res, shared=shared)
    kref = torch.zeros(64, H, D, device=dev)
    table_d = torch.from_numpy(table).to(dev, torch.int32)
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    scale = D ** -0.5
    t_write = t_attn = 0.0
    flops = 0
    for c in range(PF_CTX // PF_CHUNK):
        pos = np.arange(c * PF_CHUNK, (c + 1) * PF_CHUNK)
        slots = np.concatenate([table[s][pos // BS] * BS + pos % BS for s in range(PF_SEQS)])
        plan = shared.planner.plan(slots)
        opened = store.prepare(plan, 4)
        shared.commit(plan)
        meta, extra = stage_plan(plan, dev, None)
        shared.apply_res_map(*extra[:4])
        if opened is not None:
            store.write_headers(torch.from_numpy(opened[0]).to(dev), torch.from_numpy(opened[1]).to(dev))
        k = torch.randn(slots.size, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
        v = torch.randn(slots.size, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
        q = torch.randn(slots.size, HQ, D, device=dev, dtype=torch.bfloat16, generator=gen)
        out = torch.empty_like(q)
        ctx = (c + 1) * PF_CHUNK
        prefill = [(s * PF_CHUNK, (s + 1) * PF_CHUNK, ctx, 0) for s in range(PF_SEQS)]
        req = list(range(PF_SEQS))
        plan_d = pf.build_dense_plan(prefill, req, HQ // H, dev)
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        ev[0].record()
        store.apply(meta, k, v, kref)
        ev[1].record()
        ev[2].record()
        for _ in range(reps):
            pf.prefill_attention(store, q, out, prefill, req, table_d, scale, dense=plan_d)
        ev[3].record()
        torch.cuda.synchronize()
        t_write += ev[0].elapsed_time(ev[1])
        t_attn += ev[2].elapsed_time(ev[3]) / reps
        flops += prefill_flops(ctx, PF_CHUNK, PF_SEQS)
    tflops = flops / (t_attn * 1e-3) / 1e12
    return {
        "workload": "cfg3: 16 x 4096 tokens in 512-token chunks over an INT4 cache, Hq 32 / H 8 / D 128, bf16, "
                    "one layer",
        "attn_ms_per_layer": round(t_attn, 3),
        "write_ms_per_layer": round(t_write, 3),
        "tflop_per_layer": round(flops / 1e12, 4),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
                     "kernel": "pack_kernel<128> + flash_kernel<128, false, 3> per chunk (8 chunks)"},
    }


TRAFFIC_PROFILE = ROOT / "profiles" / "decode_cfg2_int4_traffic.md"


def measured_traffic() -> int | None:
    """HBM bytes of one INT4 decode layer-step (decode + merge), from the committed
    FETCH_SIZE / WRITE_SIZE passes scaled by the copy calibration (the profile's
    ``traffic_bytes_per_layer_step`` line); None when the profile is absent."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_layer_step:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


C4_LAYERS, C4_S, C4_CTX, C4_HQ = 80, 16, 32768, 64  # config 4


def run_mixed(reps: int = 20) -> dict:
    """A mixed-tier layer at config 2's shape: every context's first two thirds
    written at INT4 and the rest at INT8 (a layer the controller moved from 4 to
    8; blocks keep the tier they were opened at), decoded with each tier's
    specialised kernel -- the other tier's blocks then take the generic register
    path -- beside the same contexts stored at one tier."""
    import torch

    from echokv_amd.kernels.decode import decode_attention
    from echokv_amd.tiered_cache import TieredKVCache, TieredLayout
    from echokv_amd.write_plan import SharedState, stage_plan

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(11)
    ctx = rng.integers(512, 8193, S).astype(np.int64)
    layout = TieredLayout(H, D, BS, MEM, KG, VG)
    nbs = -(-ctx // BS)
    nb = int(nbs.sum()) + 16
    perm = rng.permutation(nb)
    table = np.zeros((S, int(nbs.max())), np.int64)
    o = 0
    for i, n in enumerate(nbs):
        table[i, :n] = perm[o : o + n]
        o += n
    gen = torch.Generator(device=dev)
    gen.manual_seed(12)
    cut = (ctx * 2 // 3 // BS) * BS  # block-aligned: the later blocks open at INT8

    def layer(parts):
        """A store written in len(parts) steps; parts = [(bits, start, end) per sequence fn]."""
        shared = SharedState(nb, BS, KG, S + 16, kref_window=64, device=dev)
        res = torch.zeros(S + 17, KG, H, D, dtype=torch.float16, device=dev)
        st = TieredKVCache(layout, layout.alloc_pages(nb, dev), residual=res, shared=shared)
        kref = torch.zeros(64, H, D, device=dev)
        for bits, lo, hi in parts:
            slots = np.concatenate([table[i][np.arange(lo[i], hi[i]) // BS] * BS + np.arange(lo[i], hi[i]) % BS
                                    for i in range(S)])
            plan = shared.planner.plan(slots)
            op = st.prepare(plan, bits)
            shared.commit(plan)
            meta, extra = stage_plan(plan, dev, None)
            shared.apply_res_map(*extra[:4])
            if op is not None:
                st.write_headers(torch.from_numpy(op[0]).to(dev), torch.from_numpy(op[1]).to(dev))
            k = torch.randn(slots.size, H, D, device=dev, dtype=torch.float16, generator=gen)
            v = torch.randn(slots.size, H, D, device=dev, dtype=torch.float16, generator=gen)
            k.view(slots.size, H * D)[:, torch.randperm(H * D, generator=gen, device=dev)[: H * D // 100]] *= 10
            st.apply(meta, k, v, kref)
            del k, v
        torch.cuda.synchronize()
        return st

    zero = np.zeros(S, np.int64)
    stores = {"mixed": layer([(4, zero, cut), (8, cut, ctx)]), "int4": layer([(4, zero, ctx)]),
              "int8": layer([(8, zero, ctx)])}
    table_d = torch.from_numpy(table).to(dev, torch.int32)
    lens_d = torch.from_numpy(ctx).to(dev)
    q = torch.randn(S, HQ, D, device=dev, dtype=torch.float16, generator=gen)
    out = torch.empty(S, HQ, D, device=dev, dtype=torch.float16)
    num_splits = max(1, min(-(-table.shape[1] // 16), 64))
    ws = (torch.empty(S, HQ, num_splits, D, device=dev), torch.empty(S, HQ, num_splits, 2, device=dev))

    def time_us(st, tier: int, invariant: bool = False, mask: int | None = None) -> float:
        tm = None if mask is None else torch.tensor([mask], dtype=torch.int32, device=dev)

        def go():
            decode_attention(st, q, table_d, lens_d, D ** -0.5, out=out, num_splits=num_splits, workspace=ws,
                             tier=tier, batch_invariant=invariant, tier_mask=tm)

        go()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            go()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    n8 = int((-(-(ctx - cut) // BS)).sum())
    mixed_bytes = int(round(alg_bytes(ctx, 4) * (1 - (ctx - cut).sum() / ctx.sum())
                            + alg_bytes(ctx, 8) * ((ctx - cut).sum() / ctx.sum())))
    r = {"workload": "cfg2 shape, one layer: 64 x ctx U[512, 8192]; mixed = first 2/3 of each context at INT4, "
                     "the rest at INT8; graph-replayed",
         "mixed_blocks": {"4": int(nbs.sum()) - n8, "8": n8},
         "mixed_alg_bytes": mixed_bytes}
    # (label, store, kernel tier, split schedule, tier mask): one pass at a tier (the
    # other tier's blocks on the generic path), or one pass per stored tier.
    cases = (("mixed, one INT4 pass, balanced", "mixed", 4, False, None),
             ("mixed, one INT8 pass, balanced", "mixed", 8, False, None),
             ("mixed, one INT4 pass, split", "mixed", 4, True, None),
             ("mixed, tier passes 4|8, split", "mixed", 4, True, 4 | 8),
             ("int4, one pass, balanced", "int4", 4, False, None),
             ("int4, one pass, split", "int4", 4, True, None),
             ("int4, tier passes (mask 4: two empty launches), split", "int4", 4, True, 4),
             ("int8, one pass, balanced", "int8", 8, False, None))
    r["decode_us"] = {}
    for label, name, tier, inv, mask in cases:
        us = time_us(stores[name], tier, inv, mask)
        b = mixed_bytes if name == "mixed" else alg_bytes(ctx, tier)
        r["decode_us"][label] = {"us": round(us, 1), "GBs": round(b / us / 1e3, 1)}
    return r


def run_d256(reps: int = 10) -> dict:
    """Head size 256 (the MFMA kernel at 128 channels, each KV head as two half-heads
    whose waves add their partial scores): one INT4 layer of 64 sequences x ctx
    U[512, 8192], H 8 / Hq 32, page block 16, K group 16, V group 32, against the same
    contexts at head size 128."""
    import torch

    from echokv_amd.kernels.decode import decode_attention
    from echokv_amd.tiered_cache import TieredKVCache, TieredLayout
    from echokv_amd.write_plan import SharedState, stage_plan

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(13)
    ctx = rng.integers(512, 8193, S).astype(np.int64)
    nbs = -(-ctx // BS)
    nb = int(nbs.sum()) + 16
    perm = rng.permutation(nb)
    table = np.zeros((S, int(nbs.max())), np.int64)
    o = 0
    for i, n in enumerate(nbs):
        table[i, :n] = perm[o : o + n]
        o += n
    gen = torch.Generator(device=dev)
    gen.manual_seed(14)
    table_d = torch.from_numpy(table).to(dev, torch.int32)
    lens_d = torch.from_numpy(ctx).to(dev)
    out = {}
    for d in (256, 128):
        layout = TieredLayout(H, d, BS, MEM, KG, VG)
        shared = SharedState(nb, BS, KG, S + 16, kref_window=64, device=dev)
        res = torch.zeros(S + 17, KG, H, d, dtype=torch.float16, device=dev)
        st = TieredKVCache(layout, layout.alloc_pages(nb, dev), residual=res, shared=shared)
        slots = np.concatenate([table[i][np.arange(n) // BS] * BS + np.arange(n) % BS for i, n in enumerate(ctx)])
        plan = shared.planner.plan(slots)
        op = st.prepare(plan, 4)
        shared.commit(plan)
        meta, extra = stage_plan(plan, dev, None)
        shared.apply_res_map(*extra[:4])
        if op is not None:
            st.write_headers(torch.from_numpy(op[0]).to(dev), torch.from_numpy(op[1]).to(dev))
        k = torch.randn(slots.size, H, d, device=dev, dtype=torch.float16, generator=gen)
        v = torch.randn(slots.size, H, d, device=dev, dtype=torch.float16, generator=gen)
        st.apply(meta, k, v, torch.zeros(64, H, d, device=dev))
        del k, v
        q = torch.randn(S, HQ, d, device=dev, dtype=torch.float16, generator=gen)
        o16 = torch.empty(S, HQ, d, device=dev, dtype=torch.float16)

        def go():
            decode_attention(st, q, table_d, lens_d, d ** -0.5, out=o16, tier=4)

        go()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            go()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        b = alg_bytes(ctx, 4) * d // D  # every per-token term scales with the head size
        out[f"D{d}"] = {"kernel": "decode_kernel<128, 4> (MFMA, split)" + (", half-heads" if d == 256 else ""),
                        "us_per_layer": round(us, 1), "GBs": round(b / us / 1e3, 1)}
        del st, shared, res
    return {"workload": "one INT4 layer, 64 x ctx U[512, 8192], H 8 / Hq 32, default (batch-invariant) schedule",
            **out}


def run_cfg4(reps: int = 5) -> dict:
    """Config 4: Llama-3.1-70B-shaped long-context decode on one GPU, no tensor
    parallelism -- 80 layers (seeded permutation of 20 INT8 / 40 INT4 / 20 INT2),
    Hq 64 / H 8 / D 128 (GQA 8), page block 16, K group 16, V group 32, mem_bits 8
    pages (about 102 GB), 16 sequences of 32768 tokens. Every layer's context is
    written through the quantize-on-write path (one synthetic K/V set, fp16
    ~N(0,1), 1% of K and of V channels x10, reused by every layer), then each tier's layers'
    decode (decode + merge) is captured as one HIP graph and replayed ``reps`` times
    between HIP events; the canary fires once over the 80 layers (8 query rows,
    the 64-key K_ref window, tiers 2 / 4 / 8), as on every 64th step."""
    import torch

    from echokv_amd.canary import canary_kl
    from echokv_amd.kernels.decode import decode_attention
    from echokv_amd.tiered_cache import TieredKVCache, TieredLayout
    from echokv_amd.write_plan import SharedState, stage_plan

    dev = torch.device("cuda:0")
    t_setup = time.time()
    rng = np.random.default_rng(3)
    tiers = rng.permutation(np.array([8] * 20 + [4] * 40 + [2] * 20))
    layout = TieredLayout(H, D, BS, MEM, KG, VG)
    page = layout.aligned_stride  # pages on 128-byte lines (see TieredLayout.alloc_pages)
    ctx = np.full(C4_S, C4_CTX, np.int64)
    nbs = -(-ctx // BS)
    nb = int(nbs.sum()) + 16
    perm = rng.permutation(nb)
    table = np.zeros((C4_S, int(nbs.max())), np.int64)
    o = 0
    for i, n in enumerate(nbs):
        table[i, :n] = perm[o : o + n]
        o += n
    shared = SharedState(nb, BS, KG, C4_S + 16, kref_window=64, device=dev)
    pre = np.concatenate([table[i][np.arange(n) // BS] * BS + np.arange(n) % BS for i, n in enumerate(ctx)])
    plan = shared.planner.plan(pre)
    print(f"[bench cfg4] planned {pre.size} slots, {time.time() - t_setup:.1f}s", file=sys.stderr, flush=True)
    stores, krefs = [], []
    for _ in range(C4_LAYERS):
        pages = layout.alloc_pages(nb, dev)
        res = torch.zeros(C4_S + 17, KG, H, D, dtype=torch.float16, device=dev)
        stores.append(TieredKVCache(layout, pages, residual=res, shared=shared))
        krefs.append(torch.zeros(64, H, D, device=dev))
    opened = [st.prepare(plan, int(t)) for st, t in zip(stores, tiers)]
    shared.commit(plan)
    meta, extra = stage_plan(plan, dev, None)
    shared.apply_res_map(*extra[:4])
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    k = torch.randn(pre.size, H, D, device=dev, dtype=torch.float16, generator=gen)
    v = torch.randn(pre.size, H, D, device=dev, dtype=torch.float16, generator=gen)
    out_ch = torch.randperm(H * D, generator=gen, device=dev)[: round(0.01 * H * D)]
    k.view(pre.size, H * D)[:, out_ch] *= 10
    v_ch = torch.randperm(H * D, generator=gen, device=dev)[: round(0.01 * H * D)]
    v.view(pre.size, H * D)[:, v_ch] *= 10
    for li, (st, op, kr) in enumerate(zip(stores, opened, krefs)):
        if op is not None:
            st.write_headers(torch.from_numpy(op[0]).to(dev), torch.from_numpy(op[1]).to(dev))
        st.apply(meta, k, v, kr)
        if li % 20 == 19:
            torch.cuda.synchronize()
            print(f"[bench cfg4] {li + 1} layers written, {time.time() - t_setup:.1f}s", file=sys.stderr, flush=True)
    del k, v
    torch.cuda.synchronize()
    setup_s = time.time() - t_setup
    print(f"[bench cfg4] state ready: {nb} blocks/layer, {nb * page * C4_LAYERS / 2**30:.1f} GiB pages, "
          f"{setup_s:.1f}s", file=sys.stderr, flush=True)

    table_d = torch.from_numpy(table).to(dev, torch.int32)
    lens_d = torch.from_numpy(ctx).to(dev)
    q = [torch.randn(C4_S, C4_HQ, D, device=dev, dtype=torch.float16, generator=gen) for _ in range(C4_LAYERS)]
    out = [torch.empty(C4_S, C4_HQ, D, device=dev, dtype=torch.float16) for _ in range(C4_LAYERS)]
    num_splits = max(1, min(-(-table.shape[1] // 16), 64))
    ws = (torch.empty(C4_S, C4_HQ, num_splits, D, device=dev), torch.empty(C4_S, C4_HQ, num_splits, 2, device=dev))
    scale = D ** -0.5
    per_tier = {}
    total_us = 0.0
    for bits in (8, 4, 2):
        layers = [li for li in range(C4_LAYERS) if tiers[li] == bits]

        def run_tier():
            for li in layers:
                decode_attention(stores[li], q[li], table_d, lens_d, scale, blocks_per_split=16, out=out[li],
                                 num_splits=num_splits, workspace=ws, tier=bits)

        run_tier()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run_tier()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
        b = alg_bytes(ctx, bits, hq=C4_HQ)
        per_tier[f"int{bits}"] = {"layers": len(layers), "us_per_layer": round(us, 1), "alg_bytes_per_layer": b,
                                  "GBs": round(b / us / 1e3, 1), "frac_of_8TBs": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        total_us += us * len(layers)
    # Canary: one fire over the 80 layers (the backend's every-64th-step probe).
    cq = torch.randn(C4_LAYERS, 8, C4_HQ, D, device=dev, dtype=torch.float16, generator=gen)
    kref = torch.randn(C4_LAYERS, 64, H, D, device=dev, generator=gen)
    canary_kl(cq, kref, (2, 4, 8), KG, scale)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        canary_kl(cq, kref, (2, 4, 8), KG, scale)
    e1.record()
    torch.cuda.synchronize()
    canary_us = e0.elapsed_time(e1) * 1e3 / reps
    step_bytes = sum(alg_bytes(ctx, int(t), hq=C4_HQ) for t in tiers)
    return {
        "workload": "cfg4: Llama-3.1-70B-shaped decode, 80 layers (20 INT8 / 40 INT4 / 20 INT2), batch 16 x 32768 "
                    "tokens, Hq 64 / H 8 / D 128, page block 16, K group 16, V group 32, mem_bits 8 pages",
        "pages_GiB": round(nb * page * C4_LAYERS / 2**30, 1),
        "decode_ms_per_step": round(total_us / 1e3, 3),
        "decode_alg_GB_per_step": round(step_bytes / 1e9, 2),
        "decode_GBs_per_step": round(step_bytes / total_us / 1e3, 1),
        "per_tier": per_tier,
        "canary_us_per_fire_80_layers": round(canary_us, 1),
        "setup_s": round(setup_s, 1),
        "data": "synthetic: fp16 K/V ~N(0,1), 1% of K and of V channels x10 (one set for all layers), random block tables",
    }


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(store, shared, q, kn, vn, table, lens) -> dict:
    """The reference's PyTorch path restated in torch (``oracle/torch_cpu.py``) on the
    host cores, on bounded samples of the benchmark's own data (one INT4 layer):

    * decode (``value``): gather + dequantize + SDPA of a sample of the batch's
      sequences, GB/s of the same algorithmic bytes as the GPU figure;
    * write: one decode step's quantize-on-write of the layer (finalize of the
      completing groups, then the 64 token rows), microseconds;
    * prefill: the last 512-token chunk of one 4096-token context (bottom-right
      causal), TFLOP/s of 4 D Hq per visible pair;
    * canary: the per-tier KL of one layer (64 K_ref keys, 4 query rows).
    """
    import torch

    from oracle import torch_cpu as TC
    from oracle.store import Layout, PageStore

    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1))
    torch.set_num_threads(threads)
    L = Layout(H, D, BS, MEM, KG, VG)
    ps = PageStore.over(L, store.pages.cpu().numpy().copy(), store.res_k.float().cpu().numpy(),
                        store.block_res.cpu().numpy(), store.res_group.cpu().numpy())
    qc = q.float().cpu()
    out = {"cores": threads, "cpu": _cpu_model(), "kind": "port"}

    # Decode: the whole layer-step (every sequence of the batch), repeated until
    # about 10 s of CPU work (at most 8 times).
    n_seq, reps, dt = S, 0, 0.0
    while reps < 8 and (reps == 0 or dt < 10.0):
        t0 = time.perf_counter()
        TC.decode(ps, qc[:n_seq], table[:n_seq], lens[:n_seq], D ** -0.5)
        dt += time.perf_counter() - t0
        reps += 1
    gbs = alg_bytes(lens[:n_seq], 4) * reps / dt / 1e9
    out["value"] = round(gbs, 3)
    out["unit"] = "GB/s"
    out["sample"] = (f"torch CPU decode of one INT4 layer-step over {n_seq} of {S} sequences "
                     f"({int(lens[:n_seq].sum())} tokens), {reps} times, {dt:.2f}s on {threads} threads")

    # Write: the next step's plan for this layer (positions lens), on the host copy.
    slots = table[np.arange(S), lens // BS] * BS + lens % BS
    plan = shared.planner.plan(slots)
    ps.apply_res_map(plan.res_map_block, plan.res_map_value, plan.res_group_slot, plan.res_group_value)
    tok = np.stack([plan.tok_slot, plan.tok_res, plan.tok_sealed, plan.tok_kref])
    kc, vc = kn.float().cpu(), vn.float().cpu()
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        TC.write_step(ps, kc, vc, tok, plan.fin)
    out["write_us_per_layer_step"] = round((time.perf_counter() - t0) / reps * 1e6, 1)
    out["write_sample"] = f"{S} token rows + {plan.n_fin} completing K groups of one layer, {reps} repeats"

    # Prefill: the last chunk of a 4096-token context, for the 8 longest sequences.
    rows = [int(r) for r in np.argsort(lens)[-8:]]
    ctx = min(int(lens[rows].min()), PF_CTX)
    pq = torch.randn(len(rows) * PF_CHUNK, HQ, D)
    chunks = [(i * PF_CHUNK, (i + 1) * PF_CHUNK, ctx, 0) for i in range(len(rows))]
    t0 = time.perf_counter()
    TC.prefill(ps, pq, chunks, rows, table, D ** -0.5)
    dt = time.perf_counter() - t0
    out["prefill_tflops"] = round(prefill_flops(ctx, PF_CHUNK, len(rows)) / dt / 1e12, 4)
    out["prefill_sample"] = f"{len(rows)} x one {PF_CHUNK}-token chunk over a {ctx}-token INT4 context, {dt:.2f}s"

    # Canary: one layer's per-tier KL.
    qr = torch.randn(4, HQ, D)
    kref = torch.randn(64, H, D)
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        TC.canary_kl(qr, kref, (2, 4, 8), KG, D ** -0.5)
    out["canary_us_per_layer"] = round((time.perf_counter() - t0) / reps * 1e6, 1)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--bps", type=int, default=16, help="blocks per decode split")
    ap.add_argument("--max-splits", type=int, default=64, help="cap on decode splits per sequence")
    ap.add_argument("--schedule", choices=("balanced", "split"), default="balanced",
                    help="decode schedule: the batch's blocks spread evenly over the GPU's workgroups, "
                         "or each sequence split by its own length (batch-invariant)")
    ap.add_argument("--reps", type=int, default=50, help="graph replays of the 16 INT4 layers' decode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-3 prefill measurement")
    ap.add_argument("--no-mixed", action="store_true", help="skip the mixed-tier layer measurement")
    ap.add_argument("--prefill-only", action="store_true", help="only the config-3 prefill measurement")
    ap.add_argument("--config4", action="store_true",
                    help="only config 4 (70B shape, 80 layers, about 102 GB of pages): decode per tier and the canary")
    ap.add_argument("--config5", action="store_true",
                    help="only config 5's stand-in (bench_e2e.py with its defaults): a random-init Llama-3.1-8B-shaped "
                         "model served through the backend at ECHOKV_MEM_BITS=4 against a dense 16-bit KV loop")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 1 GiB device-to-device 5 times (the reference kernel for FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.prefill_only:
        print(json.dumps({"prefill": run_prefill()}), flush=True)
        return
    if args.config4:
        print(json.dumps({"cfg4": run_cfg4()}), flush=True)
        return
    if args.config5:
        import bench_e2e

        print(json.dumps({"cfg5": bench_e2e.run_cfg5(bench_e2e.parser().parse_args([]))}), flush=True)
        return
    print(json.dumps(run(args)), flush=True)


def plan_only_us(n_seq: int, steps: int = 50) -> float:
    """Host time of the native planner alone (plan + commit) per decode step of
    ``n_seq`` sequences at random positions, block 16 / K group 16."""
    from echokv_amd.write_plan import SharedState

    rng = np.random.default_rng(3)
    ctx = rng.integers(512, 8193, n_seq)
    nbs = -(-(ctx + steps + 1) // BS)
    base = np.concatenate([[0], np.cumsum(nbs)[:-1]])
    sh = SharedState(int(nbs.sum()), BS, KG, n_seq + 16, kref_window=64, device="cpu")
    total = 0.0
    for i in range(steps):
        pos = ctx + i
        slots = (base + pos // BS) * BS + pos % BS
        t0 = time.perf_counter()
        sh.commit(sh.planner.plan(slots))
        total += time.perf_counter() - t0
    return round(total / steps * 1e6, 1)


def copy_ceiling(dev, nbytes: int = 1 << 30, reps: int = 10) -> float:
    """The same run's device-to-device copy rate (bytes read + written per second, GB/s):
    what a plain streaming kernel reaches on this GPU."""
    import torch

    a = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2 * nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del a, b
    return round(gbs, 1)


def copy_calibration(nbytes: int = 1 << 30, reps: int = 5) -> None:
    """A plain copy of known size: under ``rocprofv3 --pmc FETCH_SIZE`` (then WRITE_SIZE)
    it reads nbytes / 1024 KiB per dispatch, which scales the decode kernel's counters."""
    import torch

    a = torch.ones(nbytes, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "reps": reps}), flush=True)


if __name__ == "__main__":
    main()
