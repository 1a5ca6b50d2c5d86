"""GPU: the vLLM backend driven through a serving sequence with fake vLLM
objects (as tests/echokv_vllm/test_vllm_e2e.py drives the real engine): 3 layers
whose caches are views of one layer-interleaved pool, a chunked prefill (long
and short chunks), eager decode steps, then decode steps replayed from one
captured HIP graph, with the canary firing. Every layer's attention output is
checked against the float64 oracle over that layer's own page bytes, and the
canary's δ̂ against the oracle canary on the rows it stashed."""

import sys
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from echokv_amd import _vllm
from echokv_amd.backend import EchoKVAttentionImpl, EchoKVMetadataBuilder
from echokv_amd.controller import SUPPORTED_BITS
from echokv_amd.tiered_cache import TieredLayout
from gpu_util import maxdiff
from oracle import attention as OA
from oracle import canary as OC
from oracle import store as OS

pytestmark = pytest.mark.gpu

H, HQ, D, BS, KG, VG, LAYERS = 8, 32, 128, 16, 16, 32, 3
PROMPTS = [40, 150, 17, 300]
TOL = 2e-3


def oracle_of(impl):
    st = impl.store
    L = st.layout
    OL = OS.Layout(L.num_kv_heads, L.head_size, L.block_size, L.mem_bits, L.k_group, L.v_group)
    return OS.PageStore.over(OL, st.pages.cpu().numpy(), st.res_k.float().cpu().numpy(), st.block_res.cpu().numpy(),
                             st.res_group.cpu().numpy())


@pytest.fixture(params=["plain", "own-group"])
def env(monkeypatch, request):
    for k, v in {"ECHOKV_K_GROUP": "16", "ECHOKV_MEM_BITS": "8", "ECHOKV_CANARY_INTERVAL": "2",
                 "ECHOKV_KREF_WINDOW": "32", "ECHOKV_RESIDUAL_SLOTS": "24",
                 "ECHOKV_OWN_GROUP_EXACT": "1" if request.param == "own-group" else "0"}.items():
        monkeypatch.setenv(k, v)
    yield request.param == "own-group"
    _vllm.set_forward_metadata(None)


def make_engine(device, tiers):
    per_token = TieredLayout.per_token_bytes(H, D, 8, KG, VG)
    num_blocks = 128
    pool = torch.zeros(num_blocks, LAYERS, BS, per_token, dtype=torch.uint8, device=device)
    layers = []
    for li in range(LAYERS):
        impl = EchoKVAttentionImpl(HQ, D, D ** -0.5, H)
        # vLLM builds layers under the model's dtype (fp16 here): residual and stash follow it.
        impl.residual, impl.stash = impl.residual.half(), impl.stash.half()
        impl.controller.bits = tiers[li]
        layers.append(SimpleNamespace(kv_cache=pool[:, li : li + 1], impl=impl, layer_name=f"model.layers.{li}.attn"))
    cfg = SimpleNamespace(
        model_config=SimpleNamespace(max_model_len=2048, dtype=torch.float16,
                                     get_num_attention_heads=lambda pc: HQ),
        parallel_config=None, scheduler_config=SimpleNamespace(max_num_seqs=8),
        compilation_config=SimpleNamespace(max_cudagraph_capture_size=16), speculative_config=None)
    spec = SimpleNamespace(block_size=BS, num_kv_heads=H, head_size=D)
    builder = EchoKVMetadataBuilder(spec, [l.layer_name for l in layers], cfg, device)
    builder.bind_layers(layers)
    return builder, layers, pool


class CanaryCheck:
    """Snapshot what a fire step stashed (query rows, K_ref ring in ring order), then
    check the δ̂ the next build computed from it against the oracle canary."""

    def __init__(self, builder, layers):
        self.builder, self.layers = builder, layers
        self.snap = None
        self.checked = 0

    def after_step(self, md):
        if not md.fire:
            return
        torch.cuda.synchronize()
        pl = self.builder.shared.planner
        k = self.builder.canary.stashed[0]
        self.snap = []
        for l in self.layers:
            ring = l.impl.kref_buf.cpu().numpy()
            order = (np.arange(pl.kref_fill) + pl.kref_pos - pl.kref_fill) % ring.shape[0]
            self.snap.append((l.impl.stash[:k].float().cpu().numpy(), ring[order]))

    def after_build(self):
        if self.snap is None or self.builder.canary.scored is None:
            return
        deltas = self.builder.canary.scored[0].cpu().numpy()
        for li, (q, ring) in enumerate(self.snap):
            ref = OC.canary_kl(q, ring, SUPPORTED_BITS, KG, D ** -0.5)
            np.testing.assert_allclose(deltas[li], ref, rtol=2e-3, atol=2e-6)
        print(f"[backend canary] delta = {deltas[0].round(6).tolist()} (layer 0) matches the oracle", flush=True)
        self.snap = None
        self.checked += 1


class Batch:
    """The step's CommonAttentionMetadata (the fields the builder reads)."""

    def __init__(self, device, table, starts, lens, slots, n_tokens):
        self.num_reqs = len(lens)
        self.num_actual_tokens = n_tokens
        self.query_start_loc_cpu = torch.tensor(starts, dtype=torch.int32)
        self.seq_lens = torch.tensor(lens, dtype=torch.int32, device=device)
        self.seq_lens_cpu_upper_bound = None  # not a known vLLM table: the builder copies the device mapping
        self.slot_mapping = torch.tensor(slots, dtype=torch.int64, device=device)
        self.block_table_tensor = table
        self.causal = True
        self.req_idx = None


def slots_for(table_np, lens_before, counts):
    out = []
    for r, (p0, n) in enumerate(zip(lens_before, counts)):
        pos = np.arange(p0, p0 + n)
        out.append(table_np[r][pos // BS] * BS + pos % BS)
    return np.concatenate(out)


def run_layers(layers, md, q, k, v):
    _vllm.set_forward_metadata(md)
    outs = []
    for li, layer in enumerate(layers):
        out = torch.zeros(q[li].shape[0], HQ * D, device=q[li].device, dtype=torch.float16)
        layer.impl.do_kv_cache_update(layer, k[li], v[li], layer.kv_cache, md.slot_mapping)
        layer.impl.forward(layer, q[li], k[li], v[li], layer.kv_cache, md, out)
        outs.append(out)
    return outs


def check_decode(layers, table_np, lens, q, outs, label):
    worst = 0.0
    for li, layer in enumerate(layers):
        ps = oracle_of(layer.impl)
        n = len(lens)
        ref = OA.decode_attention(ps, q[li][:n].float().cpu().numpy(), table_np, np.asarray(lens), D ** -0.5,
                                  vectorized=True)
        worst = max(worst, maxdiff(outs[li].view(-1, HQ, D)[:n], ref))
    print(f"[backend {label}] max err {worst:.3e}", flush=True)
    assert worst <= TOL, f"{label}: {worst}"


def test_prefill_decode_and_graph_replayed_steps_match_the_oracle(device, env):
    rng = np.random.default_rng(12)
    builder, layers, pool = make_engine(device, tiers=[4, 8, 2])
    nreq = len(PROMPTS)
    table_np = rng.permutation(128)[: nreq * 32].reshape(nreq, 32).astype(np.int64)
    table = torch.from_numpy(table_np).to(device, torch.int32)
    gen = torch.Generator(device=device)
    gen.manual_seed(5)

    def rand(n, heads):
        return [torch.randn(n, heads, D, device=device, generator=gen).half() for _ in range(LAYERS)]

    # Step 1: the prompts as one chunked-prefill batch (long and short chunks).
    starts = np.concatenate([[0], np.cumsum(PROMPTS)])
    slots = slots_for(table_np, [0] * nreq, PROMPTS)
    md = builder.build(0, Batch(device, table, starts, PROMPTS, slots, int(starts[-1])))
    assert md.prefill is not None and md.decode is None
    # head size 256: the fused MFMA kernel at every length; 96: the fp32 kernel
    assert (md.prefill.dense is not None) == (D in (64, 128))
    q, k, v = rand(int(starts[-1]), HQ), rand(int(starts[-1]), H), rand(int(starts[-1]), H)
    outs = run_layers(layers, md, q, k, v)
    torch.cuda.synchronize()
    worst = 0.0
    for li, layer in enumerate(layers):
        ps = oracle_of(layer.impl)
        if env:  # own-group-exact prefill: each query's own K group from this step's keys
            ref = OA.prefill_own_group_exact(ps, q[li].float().cpu().numpy(), k[li].float().cpu().numpy(),
                                             md.prefill.entries, md.prefill.reqs, table_np, D ** -0.5)
        else:
            ref = OA.prefill_attention(ps, q[li].float().cpu().numpy(), md.prefill.entries, md.prefill.reqs,
                                       table_np, D ** -0.5, vectorized=True)
        worst = max(worst, maxdiff(outs[li].view(-1, HQ, D), ref))
        assert int(layer.impl.store.tag[table_np[1, 0]]) == layer.impl.controller.bits
    print(f"[backend prefill{' own-group' if env else ''}] max err {worst:.3e}", flush=True)
    assert worst <= TOL

    lens = list(PROMPTS)
    pad = 6  # a graph batch: 4 live requests + 2 padding rows

    # One block table for every decode step (as vLLM keeps its tables in fixed
    # buffers): a captured graph reads the table at the address it was captured with.
    bt = torch.cat([table, torch.zeros(pad - nreq, table.shape[1], dtype=table.dtype, device=device)])

    def decode_batch():
        slots = np.concatenate([slots_for(table_np, lens, [1] * nreq), -np.ones(pad - nreq, np.int64)])
        new_lens = [x + 1 for x in lens] + [0] * (pad - nreq)
        starts = np.arange(pad + 1)
        return Batch(device, bt, starts, new_lens, slots, pad), new_lens[:nreq]

    canary = CanaryCheck(builder, layers)

    # Steps 2-3: eager decode.
    for step in range(2):
        cm, new_lens = decode_batch()
        md = builder.build(0, cm)
        canary.after_build()
        assert md.decode is not None and md.decode.lens.shape[0] == pad and md.prefill is None
        q, k, v = rand(pad, HQ), rand(pad, H), rand(pad, H)
        outs = run_layers(layers, md, q, k, v)
        torch.cuda.synchronize()
        canary.after_step(md)
        lens = new_lens
        check_decode(layers, table_np, lens, q, outs, f"eager decode {step}")

    # Each layer's controller moves to another tier before the graph is captured:
    # the blocks opened from now on (request 3 crosses a block boundary during the
    # replayed steps) take the new tier, so the layers come to hold two tiers after
    # capture, and the replayed decode follows the step's device tier masks.
    for layer, bits in zip(layers, (8, 2, 4)):
        layer.impl.controller.bits = bits
    held_before = [sum(b for b, n in l.impl.store.pool.live_tiers().items() if n) for l in layers]

    # Steps 4-9: one graph captured at the decode shape, replayed with fresh metadata.
    sq, sk, sv = rand(pad, HQ), rand(pad, H), rand(pad, H)
    souts = [torch.zeros(pad, HQ * D, device=device, dtype=torch.float16) for _ in range(LAYERS)]
    cm, new_lens = decode_batch()
    md = builder.build(0, cm)
    canary.after_build()
    _vllm.set_forward_metadata(md)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for li, layer in enumerate(layers):
            layer.impl.do_kv_cache_update(layer, sk[li], sv[li], layer.kv_cache, md.slot_mapping)
            layer.impl.forward(layer, sq[li], sk[li], sv[li], layer.kv_cache, md, souts[li])
    for step in range(6):
        if step:
            cm, new_lens = decode_batch()
            md = builder.build(0, cm)
            canary.after_build()
        for li in range(LAYERS):
            sq[li].copy_(torch.randn(pad, HQ, D, device=device, generator=gen).half())
            sk[li].copy_(torch.randn(pad, H, D, device=device, generator=gen).half())
            sv[li].copy_(torch.randn(pad, H, D, device=device, generator=gen).half())
        graph.replay()
        torch.cuda.synchronize()
        canary.after_step(md)
        lens = new_lens
        check_decode(layers, table_np, lens, sq, souts, f"graph decode {step}")
    held_after = [sum(b for b, n in l.impl.store.pool.live_tiers().items() if n) for l in layers]
    print(f"[backend] tiers held by each layer: {held_before} before the graph, {held_after} after", flush=True)
    assert any(a & (a - 1) and not (b & (b - 1)) for a, b in zip(held_after, held_before)), \
        "a layer came to hold two tiers during the replayed steps"
    assert canary.checked >= 2, "the canary fired and was scored, eagerly and from graph-replayed steps"
    assert all(l.impl.controller.fires >= 1 for l in layers), "every controller observed a δ̂"
    for layer in layers:
        assert layer.impl.forward_calls == 4  # prefill, 2 eager decodes, the captured call; replays stay in the graph


def test_a_request_decodes_the_same_alone_and_in_a_batch(device, monkeypatch):
    """The default decode schedule is batch-invariant, as the reference's
    (docs/ECHOKV_VLLM_PLUGIN.md:118, decode.py:66-70): a request's output does not
    depend on which other requests share its step, to the bit."""
    for k, v in {"ECHOKV_K_GROUP": "16", "ECHOKV_MEM_BITS": "8", "ECHOKV_RESIDUAL_SLOTS": "24"}.items():
        monkeypatch.setenv(k, v)
    monkeypatch.delenv("ECHOKV_BATCH_INVARIANT", raising=False)
    rng = np.random.default_rng(3)
    nreq = len(PROMPTS)
    table_np = rng.permutation(128)[: nreq * 32].reshape(nreq, 32).astype(np.int64)
    table = torch.from_numpy(table_np).to(device, torch.int32)
    gen = torch.Generator(device=device)
    gen.manual_seed(9)
    total = sum(PROMPTS)
    pre = [[torch.randn(total, h, D, device=device, generator=gen).half() for _ in range(LAYERS)] for h in (HQ, H, H)]
    step = [[torch.randn(nreq, h, D, device=device, generator=gen).half() for _ in range(LAYERS)] for h in (HQ, H, H)]
    starts = np.concatenate([[0], np.cumsum(PROMPTS)])
    outs = {}
    for who in ("batch", "alone"):
        builder, layers, _ = make_engine(device, tiers=[4, 8, 2])
        md = builder.build(0, Batch(device, table, starts, PROMPTS, slots_for(table_np, [0] * nreq, PROMPTS), total))
        run_layers(layers, md, *pre)
        reqs = list(range(nreq)) if who == "batch" else [1]
        lens = [PROMPTS[r] + 1 for r in reqs]
        slots = np.concatenate([slots_for(table_np[r : r + 1], [PROMPTS[r]], [1]) for r in reqs])
        bt = table[reqs].contiguous()
        md = builder.build(0, Batch(device, bt, np.arange(len(reqs) + 1), lens, slots, len(reqs)))
        assert md.decode is not None and md.decode.batch_invariant
        outs[who] = run_layers(layers, md, *[[x[li][reqs] for li in range(LAYERS)] for x in step])
    torch.cuda.synchronize()
    for li in range(LAYERS):
        assert torch.equal(outs["batch"][li][1], outs["alone"][li][0]), f"layer {li}"
    print("[backend] request 1 decodes bit-identically alone and in a batch of 4", flush=True)
    _vllm.set_forward_metadata(None)


def test_balanced_schedule_takes_tier_passes_for_mixed_layers_in_eager_steps(device, monkeypatch):
    """ECHOKV_BATCH_INVARIANT=0 (the balanced schedule): once a layer holds blocks of
    two tiers (its controller moved, and a request opened a block at the new tier), an
    eager step decodes that layer with the split schedule's tier passes, each tier on
    its own kernel, and a layer holding one tier on that tier's balanced kernel;
    against the oracle."""
    from echokv_amd.kernels import decode as dec_mod

    for k, v in {"ECHOKV_K_GROUP": "16", "ECHOKV_MEM_BITS": "8", "ECHOKV_RESIDUAL_SLOTS": "24",
                 "ECHOKV_CANARY_INTERVAL": "1000", "ECHOKV_BATCH_INVARIANT": "0"}.items():
        monkeypatch.setenv(k, v)
    calls = []
    real = dec_mod.decode_attention

    def spy(*args, **kw):
        calls.append((kw.get("batch_invariant"), kw.get("tier_mask") is not None, kw.get("tier")))
        return real(*args, **kw)

    monkeypatch.setattr(dec_mod, "decode_attention", spy)
    rng = np.random.default_rng(21)
    builder, layers, _ = make_engine(device, tiers=[4, 8, 2])
    nreq = len(PROMPTS)
    table_np = rng.permutation(128)[: nreq * 32].reshape(nreq, 32).astype(np.int64)
    table = torch.from_numpy(table_np).to(device, torch.int32)
    gen = torch.Generator(device=device)
    gen.manual_seed(22)

    def rand(n, heads):
        return [torch.randn(n, heads, D, device=device, generator=gen).half() for _ in range(LAYERS)]

    starts = np.concatenate([[0], np.cumsum(PROMPTS)])
    md = builder.build(0, Batch(device, table, starts, PROMPTS, slots_for(table_np, [0] * nreq, PROMPTS),
                                int(starts[-1])))
    run_layers(layers, md, rand(int(starts[-1]), HQ), rand(int(starts[-1]), H), rand(int(starts[-1]), H))
    for layer, bits in zip(layers, (8, 2, 4)):  # blocks opened from now on take the new tier
        layer.impl.controller.bits = bits
    lens = list(PROMPTS)
    mixed_seen = False
    for step in range(6):  # request 3 (300 tokens) opens block 19 at its 5th step
        slots = slots_for(table_np, lens, [1] * nreq)
        lens = [x + 1 for x in lens]
        md = builder.build(0, Batch(device, table, np.arange(nreq + 1), lens, slots, nreq))
        assert md.decode is not None and not md.decode.batch_invariant
        calls.clear()
        q = rand(nreq, HQ)
        outs = run_layers(layers, md, q, rand(nreq, H), rand(nreq, H))
        torch.cuda.synchronize()
        held = [int(md.decode.host_tier_masks[l.impl.group_index]) for l in layers]
        assert len(calls) == LAYERS
        for (inv, has_mask, tier), h in zip(calls, held):
            if h & (h - 1):
                assert inv and has_mask, f"step {step}: a layer holding tiers {h} took {calls}"
                mixed_seen = True
            else:
                assert not inv and not has_mask and tier == h, f"step {step}: held {h}, call {(inv, has_mask, tier)}"
        check_decode(layers, table_np, lens, q, outs, f"balanced eager decode {step}, held {held}")
    assert mixed_seen, "a layer came to hold two tiers during the eager steps"
    _vllm.set_forward_metadata(None)


def test_serving_sequence_at_head_size_256(device, monkeypatch):
    """The same serving sequence at head size 256: decode on the MFMA kernels as
    half-heads (tier passes under graph replay included), prefill on the fused MFMA
    kernel at every chunk length, the canary at 256 channels; against the oracle."""
    for k, v in {"ECHOKV_K_GROUP": "16", "ECHOKV_MEM_BITS": "8", "ECHOKV_CANARY_INTERVAL": "2",
                 "ECHOKV_KREF_WINDOW": "32", "ECHOKV_RESIDUAL_SLOTS": "24", "ECHOKV_OWN_GROUP_EXACT": "0"}.items():
        monkeypatch.setenv(k, v)
    monkeypatch.setattr(sys.modules[__name__], "D", 256)
    try:
        test_prefill_decode_and_graph_replayed_steps_match_the_oracle(device, False)
    finally:
        _vllm.set_forward_metadata(None)


def test_serving_sequence_at_head_size_96_v_group_24(device, monkeypatch):
    """The same serving sequence at head size 96 with ECHOKV_V_GROUP=24 (a V group
    that is not a power of two, which the reference takes: it divides the head
    size): the backend selects it, the store writes it, and decode (eager and graph
    replayed, tier passes), prefill and the canary run on the fp32 kernels; against
    the oracle."""
    from echokv_amd.backend import EchoKVAttentionBackend

    for k, v in {"ECHOKV_K_GROUP": "16", "ECHOKV_MEM_BITS": "8", "ECHOKV_CANARY_INTERVAL": "2",
                 "ECHOKV_KREF_WINDOW": "32", "ECHOKV_RESIDUAL_SLOTS": "24", "ECHOKV_OWN_GROUP_EXACT": "0",
                 "ECHOKV_V_GROUP": "24"}.items():
        monkeypatch.setenv(k, v)
    assert EchoKVAttentionBackend.supports_head_size(96)
    monkeypatch.setattr(sys.modules[__name__], "D", 96)
    monkeypatch.setattr(sys.modules[__name__], "VG", 24)
    try:
        test_prefill_decode_and_graph_replayed_steps_match_the_oracle(device, False)
    finally:
        _vllm.set_forward_metadata(None)
