"""GPU: the HIP write path (write_tokens, finalize_k, seal, demotion) stores the
reference's exact page bytes for every golden script; the graph-style padded,
full-grid step stores the same bytes as plain writes; gather reads back the
reference's dequantized values bit for bit."""

import hashlib

import numpy as np
import pytest
import torch

import scripts as S
from echokv_amd.tiered_cache import TieredKVCache, TieredLayout
from gpu_util import gpu_replay, gpu_store
from host_sim import golden

pytestmark = pytest.mark.gpu

NAMES = [s.name for s in S.all_scripts()]


def _script(name):
    return next(s for s in S.all_scripts() if s.name == name)


@pytest.mark.parametrize("name", NAMES)
def test_hip_write_path_matches_reference_bytes(device, name):
    print(f"[store] {name}", flush=True)
    s = _script(name)
    g = golden(name)
    store, backing, stride, page, kref = gpu_replay(s, device)
    pages = store.pages.cpu().numpy()
    if s.full_bytes:
        bad = np.flatnonzero((pages != g["pages"]).any(axis=1))
        assert bad.size == 0, f"pages {bad.tolist()} differ"
        raw = backing.cpu().numpy()
        for b in range(s.num_blocks):  # nothing written past a page (0xAB guard)
            assert (raw[b * stride + page : (b + 1) * stride] == 0xAB).all()
    else:
        got = np.array([hashlib.sha256(pages[b].tobytes()).hexdigest() for b in range(s.num_blocks)])
        bad = np.flatnonzero(got != g["page_sha"])
        assert bad.size == 0, f"pages {bad.tolist()} differ"
    np.testing.assert_array_equal(store.block_res.cpu().numpy(), g["block_res"])
    np.testing.assert_array_equal(store.res_group.cpu().numpy(), g["res_group"])
    live = store.block_res[store.block_res >= 0]
    np.testing.assert_array_equal(store.res_k[live].cpu().numpy(), g["res_live"])
    if kref is not None:
        np.testing.assert_array_equal(kref.cpu().numpy(), g["kref"])
    tw = store.tokens_written
    counters = [tw[2], tw[4], tw[8], *(store.blocks_opened[b] for b in (2, 4, 8)), store.downgraded_blocks,
                store.demoted_blocks, store.sealed_groups, store.pool_free, store.residual_free]
    np.testing.assert_array_equal(np.array(counters), g["counters"])


def test_gather_reads_reference_values(device):
    s = _script("cfg1_int4_bs16")
    g = golden(s.name)
    store, *_ = gpu_replay(s, device)
    pos = torch.arange(64, device=device)
    table = torch.from_numpy(s.meta["table"]).to(device)
    k, v = store.gather(table[0][pos // s.bs], pos % s.bs)
    np.testing.assert_array_equal(k.cpu().numpy(), g["gather0_k"])
    np.testing.assert_array_equal(v.cpu().numpy(), g["gather0_v"])


def test_padded_full_grid_step_matches_plain_write(device):
    """As a captured decode graph runs the step (reference test_step_path.py:35-71):
    3 padding rows (slot -1, garbage K/V) and a full-grid finalize masked by the
    device count store exactly the plain writes' bytes; the K_ref ring too."""
    from echokv_amd.write_plan import stage_plan

    s = _script("step_path")
    plain, *_ = gpu_replay(s, device)
    graph, *_ = gpu_store(s, device)
    kr = torch.zeros(s.kref_window, s.h, s.d, device=device)
    gen = torch.Generator().manual_seed(0)
    for slots, bits, k, v in S.script_inputs(s):
        n = slots.size
        kp = torch.cat([torch.from_numpy(k), torch.randn(3, s.h, s.d, generator=gen) * 1e3]).to(device)
        vp = torch.cat([torch.from_numpy(v), torch.randn(3, s.h, s.d, generator=gen) * 1e3]).to(device)
        padded = torch.cat([torch.from_numpy(slots), torch.full((3,), -1, dtype=torch.int64)])
        plan = graph.planner.plan(padded)
        opened = graph.prepare(plan, bits)
        graph.shared.commit(plan)
        meta, extra = stage_plan(plan, device, opened)
        graph.shared.apply_res_map(*extra[:4])
        if opened is not None:
            graph.write_headers(extra[4], extra[5])
        graph.apply(meta, kp, vp, kref=kr, capturing=True)
        assert n + 3 == meta.n_rows
    torch.cuda.synchronize()
    assert torch.equal(plain.pages, graph.pages)
    assert torch.equal(plain.block_res, graph.block_res)
    live = plain.block_res[plain.block_res >= 0]
    assert live.numel() and torch.equal(plain.res_k[live], graph.res_k[live])
    np.testing.assert_array_equal(kr.cpu().numpy(), golden("step_path")["kref"])


def test_graph_replayed_step_matches_plain_write(device):
    """The write step captured once as a HIP graph over fixed buffers (rows padded
    to a fixed count, plan staged into the buffers before each replay, full-grid
    finalize masked by the device count) stores the plain writes' bytes."""
    from echokv_amd.write_plan import WriteMeta, stage_plan

    s = _script("step_path")
    plain, *_ = gpu_replay(s, device)
    st, *_ = gpu_store(s, device)
    steps = list(S.script_inputs(s))
    rows = max(sl.size for sl, *_ in steps) + 3
    tok = torch.full((4, rows), -1, dtype=torch.int64, device=device)
    fin = torch.zeros(rows, 3 + s.kg, dtype=torch.int64, device=device)
    cnt = torch.zeros(1, dtype=torch.int64, device=device)
    kb = torch.zeros(rows, s.h, s.d, device=device)
    vb = torch.zeros(rows, s.h, s.d, device=device)
    kr = torch.zeros(s.kref_window, s.h, s.d, device=device)
    gmeta = WriteMeta(tok=tok, fin=fin, fin_count=cnt, n_rows=rows, n_fin=rows)
    st.apply(gmeta, kb, vb, kref=kr, capturing=True)  # warm-up: every row is padding, no group completes
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st.apply(gmeta, kb, vb, kref=kr, capturing=True)
    gen = torch.Generator().manual_seed(1)
    for i, (slots, bits, k, v) in enumerate(steps):
        print(f"[store] graph replay step {i}", flush=True)
        n = slots.size
        padded = torch.cat([torch.from_numpy(slots), torch.full((rows - n,), -1, dtype=torch.int64)])
        plan = st.planner.plan(padded)
        opened = st.prepare(plan, bits)
        st.shared.commit(plan)
        meta, extra = stage_plan(plan, device, opened)
        st.shared.apply_res_map(*extra[:4])
        if opened is not None:
            st.write_headers(extra[4], extra[5])
        tok.copy_(meta.tok)
        if meta.n_fin:
            fin[: meta.n_fin].copy_(meta.fin)
        cnt.copy_(meta.fin_count)
        kb[:n].copy_(torch.from_numpy(k))
        vb[:n].copy_(torch.from_numpy(v))
        kb[n:].copy_(torch.randn(rows - n, s.h, s.d, generator=gen) * 1e3)
        vb[n:].copy_(torch.randn(rows - n, s.h, s.d, generator=gen) * 1e3)
        graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(plain.pages, st.pages)
    assert torch.equal(plain.block_res, st.block_res)
    live = plain.block_res[plain.block_res >= 0]
    assert live.numel() and torch.equal(plain.res_k[live], st.res_k[live])
    np.testing.assert_array_equal(kr.cpu().numpy(), golden("step_path")["kref"])


def test_decode_cases_store_oracle_bytes(device):
    """The decode-case stores (bf16-free, mixed tiers, pool pressure) written on the
    GPU equal the CPU oracle replay byte for byte."""
    from host_sim import replay

    for i in range(len(S.DECODE_CASES)):
        s = S.decode_case(i)
        sim = replay(s)
        store, *_ = gpu_replay(s, device)
        bad = np.flatnonzero((store.pages.cpu().numpy() != sim.ps.pages).any(axis=1))
        assert bad.size == 0, f"{s.name}: pages {bad.tolist()} differ"


VG_CASES = [
    # name, h, d, bs, mem_bits, seq lens, tier plan, k_group, v_group
    ("vg24_d96_pool", 4, 96, 32, 4, [33, 97, 128], [8, 8, 4], 32, 24),  # demotions: store_blocks
    ("vg6_d96_h16", 16, 96, 16, 8, [1, 40, 100], [8, 4, 2], 16, 6),  # 384 quads: two passes per row
    ("vg12_d96", 2, 96, 16, 8, [17, 50], [2, 8, 4], 16, 12),
    ("vg3_d96", 2, 96, 16, 8, [20, 35], [4, 2, 8], 16, 3),
    ("vg1_d96", 2, 96, 16, 8, [20, 35], [8, 2, 4], 16, 1),
    ("vg20_d80", 3, 80, 16, 8, [40, 9], [4, 8, 2], 16, 20),
    ("vg5_d80_pool", 2, 80, 16, 4, [50, 70, 20], [8, 8, 2], 16, 5),
    ("vg2_d64", 2, 64, 16, 8, [30, 3], [2, 4, 8], 16, 2),
]


@pytest.mark.parametrize("case", VG_CASES, ids=[c[0] for c in VG_CASES])
def test_v_groups_of_any_size_store_oracle_bytes_and_gather(device, case):
    """V groups that are not 4 * 2^j channels (any divisor of the head size, as the
    reference takes): the writes, demotions and gather equal the CPU oracle byte for
    byte and bit for bit."""
    from host_sim import replay

    name, h, d, bs, mem, lens, plan, kg, vg = case
    print(f"[store] {name}", flush=True)
    s = S.case_script(name, h, d, bs, mem, lens, plan, seed=4, kg=kg, vg=vg)
    sim = replay(s)
    store, *_ = gpu_replay(s, device)
    bad = np.flatnonzero((store.pages.cpu().numpy() != sim.ps.pages).any(axis=1))
    assert bad.size == 0, f"{name}: pages {bad.tolist()} differ"
    table = s.meta["table"]
    for i, n in enumerate(lens):
        pos = np.arange(n)
        blk, off = table[i][pos // bs], pos % bs
        k, v = store.gather(torch.from_numpy(blk).to(device), torch.from_numpy(off).to(device))
        rk, rv = sim.ps.gather(blk, off)
        np.testing.assert_array_equal(k.cpu().numpy(), rk)
        np.testing.assert_array_equal(v.cpu().numpy(), rv)


def slot_reuse_script():
    """Sixteen sequences decoding in lock step with staggered lengths (block 32,
    K group 16): whenever one sequence's token completes a group from the
    residual, another opens a group in the same step and takes the freed slot
    (the planner's stack hands it out next), so those rows' residual stores
    must follow the finalize's reads of that slot."""
    bs, kg, h, d = 32, 16, 2, 64
    start = np.array([15, 16, 47, 0, 31, 32, 79, 64, 15, 48, 47, 80, 63, 0, 31, 16])
    steps_n = 64
    nbs = -(-(start + steps_n) // bs)
    rng = np.random.default_rng(9)
    num_blocks = int(nbs.sum()) + 2
    perm = rng.permutation(num_blocks)
    table, o = [], 0
    for n in nbs:
        table.append(perm[o : o + n])
        o += n
    pre = np.concatenate([table[i][np.arange(n) // bs] * bs + np.arange(n) % bs for i, n in enumerate(start)])
    steps = [(pre.astype(np.int64), 4)]
    for t in range(steps_n):
        pos = start + t
        steps.append((np.array([table[i][p // bs] * bs + p % bs for i, p in enumerate(pos)], np.int64), 4))
    return S.Script("slot_reuse", h, d, bs, 8, kg, 32, num_blocks, 20, steps, seed=3, dtype="f16",
                    kref_window=32, full_bytes=False)


def test_fused_step_matches_finalize_then_write_and_oracle(device, monkeypatch):
    """The fused write step stores the bytes of the finalize-then-write pair and of
    the CPU oracle, on a script whose steps hand a slot released by a finalize to
    another group (the deferred residual stores are taken: counted on the host)."""
    from echokv_amd.kernels import write as W
    from echokv_amd.write_plan import WritePlanner
    from host_sim import replay

    s = slot_reuse_script()
    pl = WritePlanner(s.bs, s.kg, s.residual_slots, kref_window=s.kref_window, num_blocks=s.num_blocks)
    deferred = 0
    for slots, *_ in s.steps:
        plan = pl.plan(slots)
        freed = {int(x) for x in plan.fin[:, 2] if x >= 0}
        deferred += sum(int(x) in freed for x in plan.tok_res)
    assert deferred >= 10, f"the script defers only {deferred} residual stores"
    fused, *_, kref_f = gpu_replay(s, device)
    monkeypatch.setattr(W, "FUSED_MAX_K_GROUP", 0)  # the store's apply takes the two-launch pair
    pair, *_, kref_p = gpu_replay(s, device)
    torch.cuda.synchronize()
    print(f"[store] slot_reuse: {deferred} deferred residual stores", flush=True)
    assert torch.equal(fused.pages, pair.pages)
    assert torch.equal(fused.block_res, pair.block_res)
    live = fused.block_res[fused.block_res >= 0]
    assert live.numel() and torch.equal(fused.res_k[live], pair.res_k[live])
    assert torch.equal(kref_f, kref_p)
    sim = replay(s)
    bad = np.flatnonzero((fused.pages.cpu().numpy() != sim.ps.pages).any(axis=1))
    assert bad.size == 0, f"pages {bad.tolist()} differ from the oracle"
    np.testing.assert_array_equal(fused.res_k[live].float().cpu().numpy(), sim.ps.res_k[live.cpu().numpy()])


def test_batched_headers_equal_per_layer_writes(device):
    """One echokv_write_headers launch writes every layer's opened-block headers
    exactly where the per-layer index writes put them; other bytes stay as they were."""
    from echokv_amd.tiered_cache import HeaderWriter

    layout = TieredLayout(8, 128, 16, 8, 16, 32)
    rng = np.random.default_rng(5)
    stores = []
    for _ in range(3):
        pages = torch.from_numpy(rng.integers(0, 256, (40, layout.page_bytes), dtype=np.uint8)).to(device)
        stores.append(TieredKVCache(layout, pages, residual_slots=4))
    before = [s.pages.clone() for s in stores]
    ids = np.array([3, 17, 0, 39], np.int64)
    hdr = rng.integers(0, 256, (3, ids.size, 16), dtype=np.uint8)
    hw = HeaderWriter(stores)
    hw.check(ids)
    hw.write(torch.from_numpy(ids).to(device), torch.from_numpy(hdr.reshape(-1)).to(device))
    torch.cuda.synchronize()
    for li, s in enumerate(stores):
        want = before[li].clone()
        want[torch.from_numpy(ids).to(device), :16] = torch.from_numpy(hdr[li]).to(device)
        assert torch.equal(s.pages, want)
    with pytest.raises(ValueError):
        hw.check(np.array([40]))


@pytest.mark.parametrize("name", ["cfg1_int4_bs16", "cfg1_int8_bs16"])
def test_aligned_pages_hold_the_same_bytes_and_decode_the_same(device, name):
    """Pages placed with their data fields on 128-byte lines (TieredLayout.alloc_pages)
    hold the bytes of the same script written to plain pages, and decode the same output."""
    from echokv_amd.kernels import decode as dec

    print(f"[aligned pages] {name}", flush=True)
    s = next(x for x in S.all_scripts() if x.name == name)
    plain, *_ = gpu_replay(s, device)
    layout = TieredLayout(s.h, s.d, s.bs, s.mem_bits, s.kg, s.vg)
    rdt = torch.float16 if s.dtype == "f16" else torch.float32
    pages = layout.alloc_pages(s.num_blocks, device)
    pages.fill_(0xAB)  # the plain store's fill: bytes no write reaches compare equal too
    aligned = TieredKVCache(layout, pages, residual_slots=s.residual_slots, residual_dtype=rdt)
    kref = None if s.kref_window is None else torch.zeros(s.kref_window, s.h, s.d, device=device)
    for slots, bits, k, v in S.script_inputs(s):
        aligned.write(torch.from_numpy(k).to(device), torch.from_numpy(v).to(device),
                      torch.from_numpy(slots).to(device), bits, kref=kref)
    torch.cuda.synchronize()
    assert (aligned.pages.data_ptr() + layout.offsets["data"]) % 128 == 0
    pb = layout.page_bytes
    diff = (aligned.pages[:, :pb] != plain.pages[:, :pb]).cpu().numpy()
    rows, cols = np.nonzero(diff)
    assert rows.size == 0, f"{rows.size} bytes differ, first at blocks {rows[:8].tolist()} offsets {cols[:8].tolist()}"
    assert torch.equal(aligned.res_k, plain.res_k)
    q = torch.from_numpy(S.cfg1_query(s)).to(device)
    table = torch.from_numpy(s.meta["table"]).to(device=device, dtype=torch.int32)
    lens = torch.from_numpy(np.asarray(s.meta["lens"])).to(device)
    for bps in (1, 4):
        a = dec.decode_attention(aligned, q, table, lens, s.d ** -0.5, blocks_per_split=bps)
        b = dec.decode_attention(plain, q, table, lens, s.d ** -0.5, blocks_per_split=bps)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"{name} bps={bps}"
