"""BASELINE config 5 on one MI355X without vLLM: end-to-end decode throughput of a
random-init Llama-3.1-8B-shaped bf16 model served through the EchoKV backend,
against the same model over a dense 16-bit KV cache (a stand-in for vLLM's stock
backend, which is not importable on this machine), at the same KV byte budget.

The harness mirrors ``evaluation/serving/echokv_throughput.py:30-78``: 256
prompts of 1024 random token ids (seed 0, ids in [100, vocab - 100)), 256 greedy
output tokens each (no end of sequence), an 8 GiB KV budget, block size 64,
``ECHOKV_MEM_BITS=4`` with the live controller and canary for EchoKV. It reports
output tokens/s, KV capacity in tokens, the tier vector and stored bits at the
end, and the decode time of every layer over the last decode batch, with each
layer's stored-tier mix.

What stands in for vLLM (the same for both systems, so only attention and the KV
cache differ):

* the model: 32 decoder layers, hidden 4096, 32 query / 8 KV heads of 128,
  SwiGLU 14336, vocab 128256, RMSNorm, rotary embeddings (theta 500000), weights
  drawn N(0, 0.02) in bf16 (no checkpoint is available offline);
* the scheduler: continuous batching in the engine's order. A request is admitted
  when its whole footprint (prompt + outputs) fits the KV budget, so nothing is
  ever preempted; admitted prompts are prefilled whole, up to 8192 tokens a step;
  otherwise every running request decodes one token a step;
* every step is launched eagerly, one kernel at a time, decode steps padded to a
  multiple of 8 rows (as vLLM pads a graph batch). ``--graphs`` replays each
  padded decode size from one HIP graph instead, as vLLM's full graphs do; that
  mode is not measured yet: its first two runs faulted on tensors the captured
  graphs read after Python had freed them (the step's row index, then each
  request's newest token); both are fixed in this file and the mode awaits a run.

EchoKV runs through the product path: ``EchoKVMetadataBuilder.build`` once per
step over fake ``CommonAttentionMetadata`` (with a host block table registered as
vLLM's V1 runner registers its own, so the slot mapping is derived on the host),
then ``EchoKVAttentionImpl.do_kv_cache_update`` and ``forward`` per layer.

The stock stand-in keeps a dense cache per request slot: K stored transposed
``[slots, 8, 128, L]`` and V ``[slots, 8, L, 128]`` (bf16), L = 1280; decode is two
batched matmuls over contiguous operands with a length mask, prefill is SDPA
(flash or memory-efficient kernels only) per prompt.

    python bench_e2e.py                 # both systems, one JSON line
    python bench_e2e.py --system echokv --prompts 64
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path
from types import SimpleNamespace

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

VOCAB, HID, LAYERS, HQ, HKV, HD, FFN = 128256, 4096, 32, 32, 8, 128, 14336
EPS, THETA = 1e-5, 500000.0
GIB = 1 << 30


def log(msg: str) -> None:
    print(f"[e2e] {msg}", file=sys.stderr, flush=True)


# ---- the model ------------------------------------------------------------------------

class Model:
    """Llama-3.1-8B-shaped decoder over flattened tokens; attention is pluggable."""

    def __init__(self, dev, seed: int = 0, max_pos: int = 4096):
        import torch

        g = torch.Generator(device=dev)
        g.manual_seed(seed)

        def rnd(*shape):
            return torch.randn(*shape, generator=g, device=dev, dtype=torch.bfloat16) * 0.02

        ones = lambda: torch.ones(HID, device=dev, dtype=torch.bfloat16)  # noqa: E731
        self.embed = rnd(VOCAB, HID)
        self.layers = [SimpleNamespace(ln1=ones(), wqkv=rnd((HQ + 2 * HKV) * HD, HID), wo=rnd(HID, HQ * HD),
                                       ln2=ones(), w13=rnd(2 * FFN, HID), w2=rnd(HID, FFN)) for _ in range(LAYERS)]
        self.norm = ones()
        self.lm_head = rnd(VOCAB, HID)
        inv = 1.0 / (THETA ** (torch.arange(0, HD, 2, device=dev, dtype=torch.float32) / HD))
        ang = torch.arange(max_pos, device=dev, dtype=torch.float32)[:, None] * inv[None]
        self.cos, self.sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)

    def rope(self, x, cos, sin):
        half = HD // 2
        x1, x2 = x[..., :half], x[..., half:]
        return torch_cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin))

    def forward(self, ids, pos, attn, rows):
        """Greedy next token of the rows ``rows`` (each request's last token)."""
        import torch
        import torch.nn.functional as F

        t = ids.shape[0]
        x = self.embed[ids]
        cos, sin = self.cos[pos][:, None], self.sin[pos][:, None]
        for li, w in enumerate(self.layers):
            h = F.rms_norm(x, (HID,), w.ln1, EPS)
            q, k, v = F.linear(h, w.wqkv).split([HQ * HD, HKV * HD, HKV * HD], -1)
            q = self.rope(q.view(t, HQ, HD), cos, sin)
            k = self.rope(k.view(t, HKV, HD), cos, sin)
            o = attn(li, q, k, v.view(t, HKV, HD))
            x = x + F.linear(o, w.wo)
            h = F.rms_norm(x, (HID,), w.ln2, EPS)
            gate, up = F.linear(h, w.w13).chunk(2, -1)
            x = x + F.linear(F.silu(gate) * up, w.w2)
        h = F.rms_norm(x[rows], (HID,), self.norm, EPS)
        return torch.argmax(F.linear(h, self.lm_head), -1)


def torch_cat(parts):
    import torch

    return torch.cat(parts, -1)


# ---- EchoKV through the backend --------------------------------------------------------

class HostBlockTable:
    """What vLLM's V1 ``BlockTable`` exposes to host_slots: a host table indexed by batch
    row and its device copy (registered on construction by ``host_slots.install_v1``)."""

    def __init__(self, rows: int, cols: int, block_size: int, dev):
        import torch

        self.block_size, self.dcp_world_size, self.pcp_world_size = block_size, 1, 1
        self.block_table = SimpleNamespace(np=np.zeros((rows, cols), np.int32),
                                           gpu=torch.zeros(rows, cols, dtype=torch.int32, device=dev))


class EchoKVSystem:
    name = "echokv"

    def __init__(self, dev, budget: int, block_size: int, max_len: int, cap: int, max_seqs: int):
        import torch

        from echokv_amd import _vllm, host_slots
        from echokv_amd.backend import EchoKVAttentionImpl, EchoKVMetadataBuilder
        from echokv_amd.config import load_config
        from echokv_amd.tiered_cache import TieredLayout

        self.torch, self.vllm = torch, _vllm
        self.dev, self.bs = dev, block_size
        cfg = load_config()
        per_token = TieredLayout.per_token_bytes(HKV, HD, cfg.mem_bits, cfg.k_group, cfg.v_group)
        self.num_blocks = budget // (per_token * block_size * LAYERS)
        self.capacity_tokens = self.num_blocks * block_size
        self.layers = []
        for li in range(LAYERS):
            impl = EchoKVAttentionImpl(HQ, HD, HD ** -0.5, HKV)
            impl.residual, impl.stash = impl.residual.bfloat16(), impl.stash.bfloat16()  # the model's dtype
            kv = torch.zeros(self.num_blocks, 1, block_size, per_token, dtype=torch.uint8, device=dev)
            self.layers.append(SimpleNamespace(kv_cache=kv, impl=impl, layer_name=f"model.layers.{li}.self_attn.attn"))
        vc = SimpleNamespace(
            model_config=SimpleNamespace(max_model_len=max_len, dtype=torch.bfloat16,
                                         get_num_attention_heads=lambda pc: HQ),
            parallel_config=None, scheduler_config=SimpleNamespace(max_num_seqs=max_seqs),
            compilation_config=SimpleNamespace(max_cudagraph_capture_size=cap), speculative_config=None)
        spec = SimpleNamespace(block_size=block_size, num_kv_heads=HKV, head_size=HD)
        self.builder = EchoKVMetadataBuilder(spec, [l.layer_name for l in self.layers], vc, dev)
        self.builder.bind_layers(self.layers)
        host_slots.install_v1(HostBlockTable)
        self.table = HostBlockTable(max_seqs + 8, -(-max_len // block_size), block_size, dev)
        self.free = list(range(self.num_blocks))[::-1]
        self.blocks: dict = {}
        self.finished_blocks: dict = {}  # pages stay intact until reused: the last finished requests' blocks
        self.table_rows: tuple = ()
        self.md = None

    # scheduling
    def blocks_for(self, n_tokens: int) -> int:
        return -(-n_tokens // self.bs)

    def can_admit(self, n_tokens: int, running: int) -> bool:
        return len(self.free) >= self.blocks_for(n_tokens)

    def admit(self, req: int, n_tokens: int) -> None:
        self.blocks[req] = [self.free.pop() for _ in range(self.blocks_for(n_tokens))]

    def finish(self, req: int) -> None:
        blocks = self.blocks.pop(req)
        self.finished_blocks[req] = blocks
        self.free.extend(reversed(blocks))

    # a step
    def begin(self, reqs: list, qlens: list, lens: list, n_tokens: int) -> None:
        """Build the step's metadata: batch row i = reqs[i] (None = graph padding, no
        query token and length 0, as vLLM pads a graph batch)."""
        torch = self.torch
        t = self.table.block_table
        rows = len(reqs)
        if tuple(reqs) != self.table_rows:  # the block table follows the batch rows (vLLM's V1 runner)
            for i, r in enumerate(reqs):
                t.np[i] = 0
                if r is not None:
                    b = self.blocks[r]
                    t.np[i, : len(b)] = b
            t.gpu[:rows].copy_(torch.from_numpy(t.np[:rows]))
            self.table_rows = tuple(reqs)
        qsl = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
        cm = SimpleNamespace(num_reqs=rows, num_actual_tokens=n_tokens,
                             query_start_loc_cpu=torch.from_numpy(qsl),
                             seq_lens_cpu_upper_bound=torch.tensor(lens, dtype=torch.int32),
                             seq_lens=None, slot_mapping=None, block_table_tensor=t.gpu[:rows], causal=True,
                             req_idx=None)
        self.md = self.builder.build(0, cm)
        self.vllm.set_forward_metadata(self.md)

    def attn(self, li, q, k, v):
        layer = self.layers[li]
        out = self.torch.empty(q.shape[0], HQ * HD, device=q.device, dtype=q.dtype)
        layer.impl.do_kv_cache_update(layer, k, v, layer.kv_cache, None)
        layer.impl.forward(layer, q, k, v, layer.kv_cache, self.md, out)
        return out

    def state(self) -> dict:
        st = {"tier_vector": [l.impl.controller.bits for l in self.layers]}
        written = {b: sum(l.impl.store.tokens_written[b] for l in self.layers) for b in (2, 4, 8)}
        total = sum(written.values())
        st["tokens_written"] = {str(b): n for b, n in written.items()}
        st["avg_stored_bits"] = round(sum(b * n for b, n in written.items()) / total, 3) if total else None
        st["live_blocks_per_tier"] = [l.impl.store.pool.live_tiers() for l in self.layers]
        st["canary_fires"] = [l.impl.controller.fires for l in self.layers]
        st["ema_layer0"] = {str(b): (None if v is None else round(v, 6))
                            for b, v in self.layers[0].impl.controller.ema.items()}
        return st


# ---- the dense 16-bit stand-in ------------------------------------------------------------

class DenseSystem:
    name = "dense-bf16"

    def __init__(self, dev, budget: int, max_len: int):
        import torch

        self.torch, self.dev = torch, dev
        per_token = LAYERS * HKV * HD * 2 * 2
        self.capacity_tokens = budget // per_token
        self.lmax = max_len
        self.slots = self.capacity_tokens // max_len
        n = self.slots
        self.kt = [torch.zeros(n, HKV, HD, max_len, dtype=torch.bfloat16, device=dev) for _ in range(LAYERS)]
        self.v = [torch.zeros(n, HKV, max_len, HD, dtype=torch.bfloat16, device=dev) for _ in range(LAYERS)]
        self.free = list(range(n))[::-1]
        self.slot_of: dict = {}
        self.ar = torch.arange(max_len, device=dev)
        self.mode = None

    def can_admit(self, n_tokens: int, running: int) -> bool:
        return bool(self.free) and n_tokens <= self.lmax

    def admit(self, req: int, n_tokens: int) -> None:
        self.slot_of[req] = self.free.pop()

    def finish(self, req: int) -> None:
        self.free.append(self.slot_of.pop(req))

    def begin_prefill(self, reqs, lens):
        self.mode = ("prefill", [self.slot_of[r] for r in reqs], lens)

    def begin_decode(self, rows: int, pos_buf):
        """Decode over slots [0, rows): a row per slot (idle slots attend to position 0)."""
        self.mode = ("decode", rows, pos_buf)

    def attn(self, li, q, k, v):
        torch = self.torch
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel

        kind = self.mode[0]
        if kind == "decode":
            rows, pos = self.mode[1], self.mode[2][: self.mode[1]]
            r = torch.arange(rows, device=q.device)
            self.kt[li][r, :, :, pos] = k
            self.v[li][r, :, pos] = v
            mask = self.ar[None, :] <= pos[:, None]  # [rows, L]
            s = torch.matmul(q.view(rows, HKV, HQ // HKV, HD), self.kt[li][:rows]).float() * HD ** -0.5
            s = s.masked_fill(~mask[:, None, None, :], float("-inf"))
            p = torch.softmax(s, -1).to(torch.bfloat16)
            return torch.matmul(p, self.v[li][:rows]).reshape(rows, HQ * HD)
        out = torch.empty(q.shape[0], HQ * HD, device=q.device, dtype=q.dtype)
        o = 0
        for slot, n in zip(self.mode[1], self.mode[2]):
            kk, vv = k[o : o + n], v[o : o + n]
            self.kt[li][slot, :, :, :n] = kk.permute(1, 2, 0)
            self.v[li][slot, :, :n] = vv.transpose(0, 1)
            qq = q[o : o + n].transpose(0, 1)[None]
            ke = kk.transpose(0, 1).repeat_interleave(HQ // HKV, 0)[None]
            ve = vv.transpose(0, 1).repeat_interleave(HQ // HKV, 0)[None]
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                oo = F.scaled_dot_product_attention(qq, ke, ve, is_causal=True)
            out[o : o + n] = oo[0].transpose(0, 1).reshape(n, HQ * HD)
            o += n
        return out


# ---- the engine ---------------------------------------------------------------------------

def serve(system, model, dev, prompts: np.ndarray, out_len: int, budget_tokens: int, max_seqs: int, graphs: dict,
          echo: bool, use_graphs: bool = False) -> dict:
    """Serve every prompt to ``out_len`` greedy tokens; returns timing and counts.
    ``use_graphs``: replay decode steps from HIP graphs (one per padded batch size)
    instead of launching them eagerly."""
    import torch

    n_req, plen = prompts.shape
    waiting = list(range(n_req))
    running: list = []  # request ids in batch order
    made = np.zeros(n_req, np.int64)  # output tokens so far
    lens = np.zeros(n_req, np.int64)  # tokens in the cache
    # Every tensor a captured graph reads or writes outlives every serve() call that
    # replays it: they live in ``graphs`` (allocated once per system, at the largest size).
    last = graphs["last"]  # each request's newest token, + one row that graph padding writes
    if last.numel() < n_req + 1:
        raise ValueError("graphs['last'] must hold a row per request plus one")
    last.zero_()
    prompts_d = torch.from_numpy(prompts).to(dev)
    req_buf, pos_buf = graphs["req_buf"], graphs["pos_buf"]
    steps = dict(prefill=0, decode=0, max_running=0, graph_captures=0)
    last_batch = None
    t0 = time.perf_counter()
    while waiting or running:
        admit = []
        while (waiting and len(running) + len(admit) < max_seqs and (len(admit) + 1) * plen <= budget_tokens
               and system.can_admit(plen + out_len, len(running) + len(admit))):
            r = waiting.pop(0)
            system.admit(r, plen + out_len)
            admit.append(r)
        if admit:  # a prefill step: the admitted prompts, whole
            ids = prompts_d[admit].reshape(-1)
            pos = torch.arange(plen, device=dev).repeat(len(admit))
            rows = torch.arange(1, len(admit) + 1, device=dev) * plen - 1
            if echo:
                system.begin(admit, [plen] * len(admit), [plen] * len(admit), plen * len(admit))
            else:
                system.begin_prefill(admit, [plen] * len(admit))
            nxt = model.forward(ids, pos, system.attn, rows)
            last[torch.tensor(admit, device=dev)] = nxt
            for r in admit:
                lens[r] = plen
                made[r] = 1
            running += admit
            steps["prefill"] += 1
        else:  # a decode step of every running request
            if echo:
                b = len(running)
                rows = -(-b // 8) * 8
                reqs = running + [None] * (rows - b)
                req_ids = np.array(running + [last.numel() - 1] * (rows - b), np.int64)
                pos_np = np.array([lens[r] for r in running] + [0] * (rows - b), np.int64)
                system.begin(reqs, [1] * b + [0] * (rows - b), [int(lens[r]) + 1 for r in running] + [0] * (rows - b),
                             rows)
            else:
                hi = max(system.slot_of[r] for r in running) + 1
                rows = -(-hi // 8) * 8
                rows = min(rows, system.slots)
                by_slot = {system.slot_of[r]: r for r in running}
                req_ids = np.array([by_slot.get(s, last.numel() - 1) for s in range(rows)], np.int64)
                pos_np = np.array([lens[by_slot[s]] if s in by_slot else 0 for s in range(rows)], np.int64)
                system.begin_decode(rows, pos_buf)
            req_buf[:rows].copy_(torch.from_numpy(req_ids), non_blocking=True)
            pos_buf[:rows].copy_(torch.from_numpy(pos_np), non_blocking=True)
            def run(rows=rows):
                # The row index is made inside the step: under capture it is a node of
                # the graph, not a tensor that could be freed before a replay reads it.
                ar = torch.arange(rows, device=dev)
                nxt = model.forward(last[req_buf[:rows]], pos_buf[:rows], system.attn, ar)
                last[req_buf[:rows]] = nxt

            g = graphs.get(rows)
            if not use_graphs:
                run()
            elif g is None:
                run()  # this step, eagerly (also the warm-up of the capture)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    run()
                graphs[rows] = g
                steps["graph_captures"] += 1
            else:
                g.replay()
            for r in running:
                lens[r] += 1
                made[r] += 1
            steps["decode"] += 1
            last_batch = (list(running), [int(lens[r]) for r in running])
        steps["max_running"] = max(steps["max_running"], len(running))
        done = [r for r in running if made[r] >= out_len]
        for r in done:
            system.finish(r)
        running = [r for r in running if made[r] < out_len]
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return dict(wall_s=round(wall, 3), output_tok_s=round(int(made.sum()) / wall, 1),
                total_tok_s=round((int(made.sum()) + n_req * plen) / wall, 1), **steps), last_batch


def layer_decode_us(system, last_batch, reps: int = 5) -> list:
    """Each layer's decode (decode + merge) over the last decode batch's final state,
    at the kernel the layer runs (its controller's tier) and at the tier most of its
    blocks are stored at."""
    import torch

    from echokv_amd.kernels.decode import decode_attention

    reqs, lens = last_batch
    dev = system.dev
    table_np = np.zeros((len(reqs), system.table.block_table.np.shape[1]), np.int32)
    used = []
    for i, (r, n) in enumerate(zip(reqs, lens)):
        b = system.finished_blocks[r]
        table_np[i, : len(b)] = b
        used += b[: -(-n // system.bs)]
    used = np.array(used, np.int64)
    table = torch.from_numpy(table_np).to(dev)
    lens_d = torch.tensor(lens, dtype=torch.int64, device=dev)
    q = torch.randn(len(reqs), HQ, HD, device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    res = []
    for li, layer in enumerate(system.layers):
        store = layer.impl.store
        tags = store.pool.tag_h[used]
        mix = {b: int((tags == b).sum()) for b in (2, 4, 8)}
        entry = {"layer": li, "blocks_per_tier": mix, "controller_tier": layer.impl.controller.bits}
        for label, tier in (("us_at_controller_tier", layer.impl.controller.bits),
                            ("us_at_majority_tier", max(mix, key=mix.get))):
            for _ in range(2):
                decode_attention(store, q, table, lens_d, HD ** -0.5, out=out, tier=tier)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                decode_attention(store, q, table, lens_d, HD ** -0.5, out=out, tier=tier)
            e1.record()
            torch.cuda.synchronize()
            entry[label] = round(e0.elapsed_time(e1) / reps * 1e3, 1)
        res.append(entry)
    return res


def run_system(which: str, args) -> dict:
    import torch

    dev = torch.device("cuda:0")
    budget = int(args.kv_gib * GIB)
    max_len = args.input_len + args.output_len
    rng = np.random.default_rng(0)
    prompts = rng.integers(100, VOCAB - 100, (args.prompts, args.input_len)).astype(np.int64)
    t = time.time()
    model = Model(dev, seed=1, max_pos=max_len + 64)
    torch.cuda.synchronize()
    log(f"{which}: model ready in {time.time() - t:.1f}s")
    echo = which == "echokv"
    if echo:
        system = EchoKVSystem(dev, budget, args.block_size, max_len + 64, cap=args.max_seqs, max_seqs=args.max_seqs)
    else:
        system = DenseSystem(dev, budget, max_len)
    rows = max(args.max_seqs, 8) + 8
    graphs = {"last": torch.zeros(max(args.prompts, args.warm_prompts) + 1, dtype=torch.int64, device=dev),
              "req_buf": torch.zeros(rows, dtype=torch.int64, device=dev),
              "pos_buf": torch.zeros(rows, dtype=torch.int64, device=dev)}
    res = {"system": system.name, "kv_capacity_tokens": int(system.capacity_tokens)}
    warm, _ = serve(system, model, dev, prompts[: args.warm_prompts], args.output_len, args.max_tokens,
                    args.max_seqs, graphs, echo, args.graphs)
    log(f"{which}: warm-up {warm}")
    timed, last_batch = serve(system, model, dev, prompts, args.output_len, args.max_tokens, args.max_seqs, graphs,
                              echo, args.graphs)
    log(f"{which}: {timed}")
    res.update(timed)
    res["warmup"] = warm
    if echo:
        res["state"] = system.state()
        if args.layer_times and last_batch is not None:
            # The last decode batch has finished; its pages are intact (nothing reused them).
            res["layer_decode_us"] = layer_decode_us(system, last_batch)
    del model, system
    torch.cuda.empty_cache()
    return res


def parser() -> argparse.ArgumentParser:
    ap = argparse.ArgumentParser()
    ap.add_argument("--system", choices=("both", "echokv", "dense"), default="both")
    ap.add_argument("--prompts", type=int, default=256)
    ap.add_argument("--input-len", type=int, default=1024)
    ap.add_argument("--output-len", type=int, default=256)
    ap.add_argument("--kv-gib", type=float, default=8.0)
    ap.add_argument("--block-size", type=int, default=64)
    ap.add_argument("--max-seqs", type=int, default=256)
    ap.add_argument("--max-tokens", type=int, default=8192, help="prefill tokens per step")
    ap.add_argument("--warm-prompts", type=int, default=16)
    ap.add_argument("--no-layer-times", dest="layer_times", action="store_false")
    ap.add_argument("--graphs", action="store_true",
                    help="replay decode steps from HIP graphs (not run on the GPU yet: see the module docstring)")
    return ap


def run_cfg5(args) -> dict:
    """Both systems (or the one ``args.system`` names) on the cfg5 workload; the
    result dict that ``main`` prints (``bench.py --config5`` runs it with the defaults)."""
    os.environ.setdefault("ECHOKV_MEM_BITS", "4")
    out = {"workload": f"cfg5 stand-in: {args.prompts} x ({args.input_len} in, {args.output_len} out), greedy, "
                       f"{args.kv_gib:g} GiB KV, block {args.block_size}, random-init bf16 Llama-3.1-8B shape, "
                       f"decode steps {'graph-replayed' if args.graphs else 'eager'}",
           "echokv_env": {k: v for k, v in os.environ.items() if k.startswith("ECHOKV_")}}
    for which in (("echokv", "dense") if args.system == "both" else (args.system,)):
        out[which] = run_system(which, args)
    if "echokv" in out and "dense" in out:
        out["speedup_output_tok_s"] = round(out["echokv"]["output_tok_s"] / out["dense"]["output_tok_s"], 3)
        out["capacity_ratio"] = round(out["echokv"]["kv_capacity_tokens"] / out["dense"]["kv_capacity_tokens"], 3)
    return out


def main():
    print(json.dumps(run_cfg5(parser().parse_args())), flush=True)


if __name__ == "__main__":
    main()
