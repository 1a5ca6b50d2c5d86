"""GPU parity at the benchmark configurations' own shapes, and on the kernel
paths small cases never reach (tests/echokv_vllm/test_decode_kernel.py:69-75
runs the 8B shape the same way).

Each store is written through the product's own write path (planner + HIP
write kernels); the oracle then reads the device's page bytes (copied to the
host) and computes attention in float64. Every test prints its worst error
against the 2e-3 budget, so the margin is visible in the log.

* cfg2: one full layer per tier -- 64 sequences, contexts U[512, 8192] (seed 1),
  H 8 / D 128 / block 16 / K group 16 / V group 32, fp16 K/V with 1% of K
  channels x10, the context then one decode-step write -- decoded with fp16 and
  bf16 queries and through the generic (other-tier) path.
* cfg3: 2 sequences x 4096 tokens written in 512-token chunks, INT4, bf16
  K/V/Q and residual: every stored code and statistic byte-exact against the
  vectorized quantization, and chunked-prefill attention of the first and last
  chunks (two-pass path) plus a short tail chunk (fused path).
* cfg4 shape: GQA 8 (Hq 64), one 32k-token sequence: default splits, a split of
  more than 64 blocks (the chunk loop), more than 64 splits (the two-pass merge);
  the canary at Hq 64.
* more than 64 sequences (the chunked work-item scan; short sequences, so the
  balanced schedule's ranges cover several sequences each), V groups of 16 and 64,
  head size 64, and a layer view whose pages span more than 4 GiB (64-bit page
  addressing, as in a layer view of a pool interleaved across layers).
"""

import numpy as np
import pytest
import torch

from echokv_amd import _lib
from echokv_amd.canary import canary_kl
from echokv_amd.kernels import decode as dec
from echokv_amd.kernels import prefill as pf
from echokv_amd.tiered_cache import TieredKVCache, TieredLayout
from gpu_util import maxdiff
from oracle import attention as OA
from oracle import canary as OC
from oracle import quant as Q
from oracle import store as OS

pytestmark = pytest.mark.gpu

TOL = 2e-3


def oracle_view(store) -> OS.PageStore:
    """The oracle over a copy of a device store's bytes and residual state."""
    L = store.layout
    OL = OS.Layout(L.num_kv_heads, L.head_size, L.block_size, L.mem_bits, L.k_group, L.v_group)
    return OS.PageStore.over(OL, store.pages.cpu().numpy(), store.res_k.float().cpu().numpy(),
                             store.block_res.cpu().numpy(), store.res_group.cpu().numpy())


def block_table(rng, lens, bs, spare=16):
    """Each sequence's blocks drawn from a seeded permutation of the pages."""
    nbs = -(-(np.asarray(lens) + 1) // bs)
    nb = int(nbs.sum()) + spare
    perm = rng.permutation(nb)
    table = np.zeros((len(lens), int(nbs.max())), np.int64)
    o = 0
    for i, n in enumerate(nbs.tolist()):
        table[i, :n] = perm[o : o + n]
        o += n
    return table, nb


def slots_of(table, lens, pos_fn, bs):
    return np.concatenate([table[i][p // bs] * bs + p % bs for i, p in ((i, pos_fn(i, n)) for i, n in enumerate(lens))])


def build_layer(device, lens, bits, *, h=8, d=128, bs=16, kg=16, vg=32, mem_bits=8, dtype=torch.float16, seed=1,
                outliers=0.01, v_outliers=0.0, pages=None, table=None, v_mult=1.0):
    """A layer store written through the product path: each sequence's first
    len - 1 tokens in one step, then its last token in a second (decode) step.
    ``outliers`` / ``v_outliers``: the share of (head, channel) pairs of K / V
    scaled x10; ``v_mult``: every V value's factor."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int64)
    if table is None:
        table, nb = block_table(rng, lens, bs)
    layout = TieredLayout(h, d, bs, mem_bits, kg, vg)
    if pages is None:
        page = bs * TieredLayout.per_token_bytes(h, d, mem_bits, kg, vg)
        pages = torch.zeros(nb, page, dtype=torch.uint8, device=device)
    store = TieredKVCache(layout, pages, residual_slots=len(lens) + 16, residual_dtype=dtype)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    out_ch = torch.randperm(h * d, generator=gen, device=device)[: round(outliers * h * d)]
    v_ch = torch.randperm(h * d, generator=gen, device=device)[: round(v_outliers * h * d)]

    def kv(n):
        k = torch.randn(n, h, d, generator=gen, device=device)
        k.view(n, h * d)[:, out_ch] *= 10
        v = torch.randn(n, h, d, generator=gen, device=device) * v_mult
        v.view(n, h * d)[:, v_ch] *= 10
        return k.to(dtype), v.to(dtype)

    pre = slots_of(table, lens, lambda i, n: np.arange(n - 1), bs)
    if pre.size:
        k, v = kv(pre.size)
        store.write(k, v, torch.from_numpy(pre).to(device), bits)
    last = slots_of(table, lens, lambda i, n: np.array([n - 1]), bs)
    k, v = kv(last.size)
    store.write(k, v, torch.from_numpy(last).to(device), bits)
    torch.cuda.synchronize()
    return store, table


def check(label, got, ref, tol=TOL):
    err = maxdiff(got, ref)
    print(f"[{label}] max err {err:.3e} (budget {tol:g})", flush=True)
    assert err <= tol, f"{label}: max err {err}"
    return err


# ---- cfg2 -----------------------------------------------------------------------------

@pytest.mark.parametrize("bits", [8, 4, 2])
def test_cfg2_full_layer_decode_matches_oracle(device, bits):
    rng = np.random.default_rng(1)
    lens = rng.integers(512, 8193, 64)
    print(f"[cfg2] int{bits}: writing {int(lens.sum())} tokens", flush=True)
    store, table = build_layer(device, lens, bits, seed=1)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(11)
    q = torch.randn(64, 32, 128, device=device, generator=gen).half()
    scale = 128 ** -0.5
    for qt, name in ((q, "fp16 q"), (q.bfloat16(), "bf16 q")):
        ref = OA.decode_attention(ps, qt.float().cpu().numpy(), table, lens, scale, vectorized=True)
        got = dec.decode_attention(store, qt, table_d, lens_d, scale, tier=bits, batch_invariant=False)
        check(f"cfg2 int{bits} {name} balanced schedule", got, ref)
        got = dec.decode_attention(store, qt, table_d, lens_d, scale, tier=bits, batch_invariant=True)
        check(f"cfg2 int{bits} {name} split schedule", got, ref)
        if name == "fp16 q":  # every tile through the generic path (the layer's tier set elsewhere)
            other = 4 if bits != 4 else 8
            for inv in (False, True):
                got = dec.decode_attention(store, qt, table_d, lens_d, scale, tier=other, batch_invariant=inv)
                check(f"cfg2 int{bits} as tier {other}" + (" split schedule" if inv else ""), got, ref)


@pytest.mark.parametrize("bits", [8, 4, 2])
@pytest.mark.parametrize("span", ["short", "long"])
def test_cfg2_with_k_and_v_outliers(device, bits, span):
    """BASELINE cfg2's inputs: 1% outlier channels x10 in K and in V. Outlier V
    channels give values of magnitude 10-40 whose dequantized fp16 operand rounds
    by up to 2^-7 .. 2^-6; short contexts (few tokens, large weights) are where
    that rounding shows most in the output."""
    rng = np.random.default_rng(21)
    lens = rng.integers(16, 300, 32) if span == "short" else rng.integers(512, 8193, 64)
    store, table = build_layer(device, lens, bits, seed=21, v_outliers=0.01)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(22)
    q = torch.randn(len(lens), 32, 128, device=device, generator=gen).half()
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, 128 ** -0.5, vectorized=True)
    print(f"[cfg2 v-outliers {span} int{bits}] max |out| {np.abs(ref).max():.2f}", flush=True)
    for inv in (False, True):
        got = dec.decode_attention(store, q, table_d, lens_d, 128 ** -0.5, tier=bits, batch_invariant=inv)
        check(f"cfg2 v-outliers {span} int{bits}" + (" split schedule" if inv else ""), got, ref)
    out16 = torch.empty(len(lens), 32, 128, device=device, dtype=torch.float16)
    dec.decode_attention(store, q, table_d, lens_d, 128 ** -0.5, tier=bits, out=out16)
    raw = float(np.abs(out16.float().cpu().numpy() - ref).max())
    check(f"cfg2 v-outliers {span} int{bits} fp16 out (raw max-abs {raw:.3e})", out16, ref)


@pytest.mark.parametrize("bits", [8, 4, 2])
@pytest.mark.parametrize("gqa", [4, 7])
def test_large_v_values_stay_finite_and_accurate(device, bits, gqa):
    """V values in the thousands (V scales far above typical): where the kernel
    folds the V scale into the P operand (GQA 4 here), a tile with such scales
    rescales its weights exactly, so the operand w * s stays inside fp16; GQA 7
    takes the per-element V path. Every case is within the north-star bar scaled
    by the values' factor (the same relative accuracy as unit-scale data)."""
    rng = np.random.default_rng(31)
    lens = np.concatenate([rng.integers(1, 40, 12), rng.integers(500, 3000, 4)])
    mult = 3000.0
    store, table = build_layer(device, lens, bits, h=4, seed=31, v_mult=mult)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(32)
    q = (torch.randn(len(lens), 4 * gqa, 128, device=device, generator=gen) * 2).half()
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, 128 ** -0.5, vectorized=True)
    print(f"[large V int{bits} gqa{gqa}] max |out| {np.abs(ref).max():.1f}", flush=True)
    for inv in (False, True):
        got = dec.decode_attention(store, q, table_d, lens_d, 128 ** -0.5, tier=bits, batch_invariant=inv)
        assert torch.isfinite(got).all(), "non-finite output"
        check(f"large V int{bits} gqa{gqa}" + (" split schedule" if inv else ""), got, ref, tol=TOL * mult)


@pytest.mark.parametrize("bits", [8, 2])
def test_gqa8_on_the_int8_and_int2_kernels(device, bits):
    """GQA 8 (the 70B shape's Hq 64 / H 8) through the INT8- and INT2-specialised
    kernels, several sequences, both schedules."""
    rng = np.random.default_rng(23)
    lens = rng.integers(100, 4000, 6)
    store, table = build_layer(device, lens, bits, seed=23, v_outliers=0.01)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    gen = torch.Generator(device=device)
    gen.manual_seed(24)
    q = torch.randn(len(lens), 64, 128, device=device, generator=gen).half()
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, 128 ** -0.5, vectorized=True)
    for inv in (False, True):
        got = dec.decode_attention(store, q, table_d, torch.from_numpy(lens).to(device), 128 ** -0.5, tier=bits,
                                   batch_invariant=inv)
        check(f"gqa8 int{bits}" + (" split schedule" if inv else ""), got, ref)


# ---- cfg3 -----------------------------------------------------------------------------

def test_cfg3_chunked_prefill_bf16_writes_and_attention(device):
    h, d, bs, kg, vg, hq, seqs, ctx, chunk = 8, 128, 16, 16, 32, 32, 2, 4096, 512
    rng = np.random.default_rng(2)
    nbs = ctx // bs
    nb = seqs * nbs + 16
    table = rng.permutation(nb)[: seqs * nbs].reshape(seqs, nbs).astype(np.int64)
    layout = TieredLayout(h, d, bs, 8, kg, vg)
    page = bs * TieredLayout.per_token_bytes(h, d, 8, kg, vg)
    store = TieredKVCache(layout, torch.zeros(nb, page, dtype=torch.uint8, device=device), residual_slots=seqs + 16,
                          residual_dtype=torch.bfloat16)
    gen = torch.Generator(device=device)
    gen.manual_seed(2)
    K = torch.randn(seqs, ctx, h, d, device=device, generator=gen).bfloat16()
    V = torch.randn(seqs, ctx, h, d, device=device, generator=gen).bfloat16()
    Qr = torch.randn(seqs, ctx, hq, d, device=device, generator=gen).bfloat16()
    table_d = torch.from_numpy(table).to(device, torch.int32)
    scale = d ** -0.5
    for c in range(ctx // chunk):
        pos = np.arange(c * chunk, (c + 1) * chunk)
        slots = np.concatenate([table[s][pos // bs] * bs + pos % bs for s in range(seqs)])
        sl = slice(c * chunk, (c + 1) * chunk)
        store.write(K[:, sl].reshape(-1, h, d), V[:, sl].reshape(-1, h, d), torch.from_numpy(slots).to(device), 4)
        if c not in (0, ctx // chunk - 1):
            continue
        q = Qr[:, sl].reshape(-1, hq, d)
        n_ctx = (c + 1) * chunk
        prefill = [(s * chunk, (s + 1) * chunk, n_ctx, 0) for s in range(seqs)]
        assert pf.use_dense(prefill, d)
        out = torch.zeros(seqs * chunk, hq, d, device=device)
        pf.prefill_attention(store, q, out, prefill, [0, 1], table_d, scale)
        torch.cuda.synchronize()
        ps = oracle_view(store)
        ref = OA.prefill_attention(ps, q.float().cpu().numpy(), prefill, [0, 1], table, scale, vectorized=True)
        check(f"cfg3 chunk {c} (two-pass)", out, ref)
    # The fused path on the last 48 queries of each sequence over the full context.
    tail = 48
    q = Qr[:, ctx - tail :].reshape(-1, hq, d)
    prefill = [(s * tail, (s + 1) * tail, ctx, 0) for s in range(seqs)]
    out = torch.zeros(seqs * tail, hq, d, device=device)
    pf.prefill_attention(store, q, out, prefill, [0, 1], table_d, scale)
    torch.cuda.synchronize()
    ref = OA.prefill_attention(ps, q.float().cpu().numpy(), prefill, [0, 1], table, scale, vectorized=True)
    check("cfg3 tail (fused)", out, ref)

    # Every stored code and statistic, byte-exact (quant.py:26-75 on the bf16 inputs).
    pos = np.arange(ctx)
    blk = np.concatenate([table[s][pos // bs] for s in range(seqs)])
    off = np.concatenate([pos % bs] * seqs)
    assert (ps.pages[blk, 0] == 4).all()
    kc, vc, vs, vm, ks, km = ps.raw_vec(blk, off, 4)
    kf = K.float().cpu().numpy().reshape(-1, h, d)
    vf = V.float().cpu().numpy().reshape(-1, h, d)
    ecodes, escale, emin = Q.quantize(vf, 4, vg)
    np.testing.assert_array_equal(vc, ecodes)
    np.testing.assert_array_equal(vs.view(np.uint16), escale.view(np.uint16))
    np.testing.assert_array_equal(vm.view(np.uint16), emin.view(np.uint16))
    kgrp = kf.reshape(-1, kg, h, d)
    gsc, gmn = Q.stats_along(kgrp, 4, axis=1)
    kcodes = Q.quantize_with(kgrp, gsc[:, None], gmn[:, None], 4).reshape(-1, h, d)
    np.testing.assert_array_equal(kc, kcodes)
    np.testing.assert_array_equal(ks.view(np.uint16), np.repeat(gsc, kg, axis=0).view(np.uint16))
    np.testing.assert_array_equal(km.view(np.uint16), np.repeat(gmn, kg, axis=0).view(np.uint16))
    print(f"[cfg3] {blk.size} tokens: codes and stats byte-exact", flush=True)


# ---- cfg4 shape -----------------------------------------------------------------------

def test_cfg4_gqa8_long_context_split_paths(device):
    lens = np.array([32768])
    store, table = build_layer(device, lens, 4, seed=3)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(33)
    q = torch.randn(1, 64, 128, device=device, generator=gen).half()
    scale = 128 ** -0.5
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, scale, vectorized=True)
    nblk = -(-32768 // 16)
    for label, kw in (("balanced, 32 ranges", {}),
                      ("balanced, 2 ranges of 1024 blocks", {"num_splits": 4}),
                      ("default splits", {"batch_invariant": True}),
                      ("4 splits of 513 blocks", {"num_splits": 4, "batch_invariant": True}),
                      ("187 splits of 11 blocks", {"num_splits": 200, "blocks_per_split": 1, "batch_invariant": True})):
        got = dec.decode_attention(store, q, table_d, lens_d, scale, tier=4, **kw)
        check(f"cfg4 {label}", got, ref)
    assert -(-nblk // 4) > 64 and -(-nblk // -(-nblk // 200)) > 64


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_balanced_cost_ranges_at_every_boundary_position(device, bits):
    """The balanced schedule's ranges of equal cost (a live sequence costs its blocks
    plus its start-up) against the merge, which finds each piece's range from the
    same cost coordinate: lengths of 1 to 300 tokens around block boundaries, padding
    rows of length 0 among them, and range counts from a few (each range holding many
    sequences) to more than the batch's cost (most ranges empty). Every live row
    against the oracle; padding rows are left as they were."""
    lens_live = np.array([1, 15, 16, 17, 31, 32, 33, 47, 64, 65, 100, 129, 200, 255, 256, 257, 300, 2, 3, 48])
    store, table = build_layer(device, lens_live, bits, seed=41, v_outliers=0.01)
    ps = oracle_view(store)
    lens = lens_live.copy()
    lens[[3, 9, 15]] = 0  # padding rows
    live = lens > 0
    gen = torch.Generator(device=device)
    gen.manual_seed(42)
    q = torch.randn(len(lens), 32, 128, device=device, generator=gen).half()
    scale = 128 ** -0.5
    ref = OA.decode_attention(ps, q[torch.from_numpy(live).to(device)].float().cpu().numpy(), table[live],
                              lens[live], scale, vectorized=True)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    for ns in (1, 2, 8, 64):  # ranges are capped at S * splits / 2
        out = torch.full((len(lens), 32, 128), 7.0, device=device)
        dec.decode_attention(store, q, table_d, lens_d, scale, tier=bits, batch_invariant=False, num_splits=ns,
                             out=out)
        torch.cuda.synchronize()
        check(f"balanced int{bits}, splits {ns}", out[torch.from_numpy(live).to(device)], ref)
        assert bool((out[torch.from_numpy(~live).to(device)] == 7.0).all()), "padding rows were written"


def test_cfg4_batch_at_int4_balanced(device):
    """cfg4's decode batch at one tier: 16 sequences of 32,768 tokens, GQA 8, INT4,
    the balanced schedule (the benchmark's) and the split one, against the
    vectorized oracle."""
    lens = np.full(16, 32768)
    store, table = build_layer(device, lens, 4, seed=31, v_outliers=0.01)
    ps = oracle_view(store)
    gen = torch.Generator(device=device)
    gen.manual_seed(32)
    q = torch.randn(16, 64, 128, device=device, generator=gen).half()
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, 128 ** -0.5, vectorized=True)
    for inv in (False, True):
        got = dec.decode_attention(store, q, torch.from_numpy(table).to(device, torch.int32),
                                   torch.from_numpy(lens).to(device), 128 ** -0.5, tier=4, batch_invariant=inv)
        check("cfg4 16 x 32k int4" + (" split schedule" if inv else " balanced"), got, ref)


def test_canary_at_hq64(device):
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 8, 64, 128)).astype(np.float32)
    kref = (rng.standard_normal((2, 64, 8, 128)) * 2).astype(np.float32)
    got = canary_kl(torch.from_numpy(q).to(device).half(), torch.from_numpy(kref).to(device), (2, 4, 8), 16,
                    128 ** -0.5)
    ref = OC.canary_kl(q.astype(np.float16).astype(np.float32), kref, (2, 4, 8), 16, 128 ** -0.5)
    err = float(np.abs(got.cpu().numpy() / ref - 1).max())
    print(f"[canary hq64] max rel err {err:.3e}", flush=True)
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=2e-3, atol=2e-6)


# ---- paths small cases miss -----------------------------------------------------------

def test_more_than_64_sequences_with_padding_rows(device):
    rng = np.random.default_rng(5)
    lens = rng.integers(1, 400, 150)
    lens[[0, 1, 2, 70, 149]] = [1, 16, 17, 2, 1]
    store, table = build_layer(device, lens, 4, seed=5, outliers=0.0)
    ps = oracle_view(store)
    run = lens.copy()
    run[[3, 100]] = 0  # graph padding rows: left untouched
    gen = torch.Generator(device=device)
    gen.manual_seed(55)
    q = torch.randn(150, 32, 128, device=device, generator=gen).half()
    out = torch.full((150, 32, 128), 7.0, device=device)
    dec.decode_attention(store, q, torch.from_numpy(table).to(device, torch.int32), torch.from_numpy(run).to(device),
                         128 ** -0.5, out=out)
    split = torch.full((150, 32, 128), 7.0, device=device)
    dec.decode_attention(store, q, torch.from_numpy(table).to(device, torch.int32), torch.from_numpy(run).to(device),
                         128 ** -0.5, out=split, batch_invariant=True)
    live = np.flatnonzero(run > 0)
    ref = OA.decode_attention(ps, q[live].float().cpu().numpy(), table[live], lens[live], 128 ** -0.5,
                              vectorized=True)
    check("150 sequences", out[live], ref)
    check("150 sequences, split schedule", split[live], ref)
    assert (out[[3, 100]] == 7.0).all() and (split[[3, 100]] == 7.0).all()
    # A workspace of 6 splits: the balanced schedule's ranges fill it.
    tight = torch.full((150, 32, 128), 7.0, device=device)
    dec.decode_attention(store, q, torch.from_numpy(table).to(device, torch.int32), torch.from_numpy(run).to(device),
                         128 ** -0.5, out=tight, num_splits=6)
    check("150 sequences, 6-split workspace", tight[live], ref)
    assert (tight[[3, 100]] == 7.0).all()


@pytest.mark.parametrize("d,vg", [(128, 16), (128, 64), (64, 32), (64, 16)])
@pytest.mark.parametrize("bits", [8, 4, 2])
@pytest.mark.parametrize("h", [4, 8])
def test_v_group_and_head_size_variants(device, d, vg, bits, h):
    """Four KV heads are one decode head group, eight are two (their workgroups
    read neighbouring slices of the same token rows)."""
    lens = np.array([1, 17, 300, 64, 1000])
    store, table = build_layer(device, lens, bits, h=h, d=d, vg=vg, seed=6, outliers=0.02)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    gen = torch.Generator(device=device)
    gen.manual_seed(66)
    q = torch.randn(5, 4 * h, d, device=device, generator=gen).half()
    got = dec.decode_attention(store, q, table_d, torch.from_numpy(lens).to(device), d ** -0.5)
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, d ** -0.5, vectorized=True)
    check(f"decode H{h} D{d} VG{vg} int{bits}", got, ref)
    got = dec.decode_attention(store, q, table_d, torch.from_numpy(lens).to(device), d ** -0.5, batch_invariant=True)
    check(f"decode H{h} D{d} VG{vg} int{bits} split schedule", got, ref)
    if h == 8:
        return  # the prefill paths take the same head loop at any head count
    for path, chunk in (("dense", 100), ("fused", 30)):
        prefill, row = [], 0
        for n in lens.tolist():
            nq = min(chunk, n)
            prefill.append((row, row + nq, n, 0))
            row += nq
        qp = torch.randn(row, 4 * h, d, device=device, generator=gen).half()
        out = torch.zeros(row, 4 * h, d, device=device)
        fn = pf.prefill_attention_dense if path == "dense" else pf.prefill_attention_fused
        fn(store, qp, out, prefill, list(range(5)), table_d, d ** -0.5)
        torch.cuda.synchronize()
        ref = OA.prefill_attention(ps, qp.float().cpu().numpy(), prefill, list(range(5)), table, d ** -0.5,
                                   vectorized=True)
        check(f"prefill {path} D{d} VG{vg} int{bits}", out, ref)


@pytest.mark.parametrize("d,bs,kg,vg,h,gqa", [(96, 16, 16, 32, 4, 4), (256, 16, 16, 32, 4, 4), (256, 32, 32, 256, 2, 4),
                                               (128, 16, 8, 32, 4, 4), (128, 48, 16, 32, 4, 4), (128, 16, 16, 4, 4, 4),
                                               (80, 32, 32, 16, 4, 2), (96, 16, 16, 32, 2, 20), (96, 16, 16, 24, 4, 4),
                                               (96, 32, 32, 3, 2, 7), (80, 16, 16, 20, 2, 4)])
@pytest.mark.parametrize("bits", [8, 4, 2])
def test_layouts_outside_the_mfma_kernels(device, d, bs, kg, vg, h, gqa, bits):
    """Head sizes other than 64 / 128 / 256 (up to 256) with V groups of any size
    (24, 3, 20 channels), head size 256 with one V group per head, K groups under
    16, block sizes that are not powers of two and V groups under D/16 take the fp32
    decode kernel (the reference's PyTorch path
    serves them there), GQA 20 in two passes of query heads; prefill attends
    through decode rows (head size 256 included). Both equal the oracle."""
    lens = np.array([1, 17, 300, 64, 1000])
    store, table = build_layer(device, lens, bits, h=h, d=d, bs=bs, kg=kg, vg=vg, seed=8, outliers=0.02)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(88)
    label = f"D{d} BS{bs} KG{kg} VG{vg} H{h} GQA{gqa} int{bits}"
    q = torch.randn(5, gqa * h, d, device=device, generator=gen).half()
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, d ** -0.5, vectorized=True)
    for inv in (False, True):
        got = dec.decode_attention(store, q, table_d, lens_d, d ** -0.5, batch_invariant=inv, num_splits=3)
        check(f"decode {label}" + (" split schedule" if inv else ""), got, ref)
    prefill, row = [], 0
    for n in lens.tolist():
        nq = min(100, n)
        prefill.append((row, row + nq, n, 0))
        row += nq
    qp = torch.randn(row, gqa * h, d, device=device, generator=gen).half()
    out = torch.zeros(row, gqa * h, d, device=device)
    pf.prefill_attention(store, qp, out, prefill, list(range(5)), table_d, d ** -0.5)
    torch.cuda.synchronize()
    ref = OA.prefill_attention(ps, qp.float().cpu().numpy(), prefill, list(range(5)), table, d ** -0.5,
                               vectorized=True)
    check(f"prefill {label}", out, ref)


@pytest.mark.parametrize("h,gqa,vg,dt", [(8, 4, 32, torch.float16), (3, 4, 64, torch.bfloat16), (1, 20, 16, torch.float32),
                                         (2, 8, 128, torch.float16)])
@pytest.mark.parametrize("bits", [8, 4, 2])
def test_head_size_256_as_half_heads(device, h, gqa, vg, dt, bits):
    """Head size 256 on the 128-channel MFMA kernels: each KV head's channel halves on
    two waves that add their partial scores before the softmax. Even and odd KV head
    counts (H 3 and H 1: a workgroup's last two waves are past the last head and
    still meet every score exchange), GQA 20 (two passes of query heads), V groups
    of 16 (every tile on the register path) to 128, fp16 / bf16 / float32 queries,
    K / V and residual (the open K groups), a 2500-token sequence in one span (the
    64-block chunk loop); both schedules against the oracle, and a sequence decoded
    alone equal to itself in the batch (split schedule)."""
    lens = np.array([1, 17, 300, 64, 1000, 2500])
    store, table = build_layer(device, lens, bits, h=h, d=256, vg=vg, dtype=dt, seed=9, outliers=0.02,
                               v_outliers=0.01)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(99)
    q = torch.randn(len(lens), gqa * h, 256, device=device, generator=gen).to(dt)
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, 256 ** -0.5, vectorized=True)
    label = f"D256 H{h} GQA{gqa} VG{vg} {str(dt)[6:]} int{bits}"
    got = dec.decode_attention(store, q, table_d, lens_d, 256 ** -0.5, tier=bits, batch_invariant=False)
    check(f"{label} balanced", got, ref)
    for ns in (None, 1):
        got = dec.decode_attention(store, q, table_d, lens_d, 256 ** -0.5, tier=bits, num_splits=ns)
        check(f"{label} split, splits {ns or 'default'}", got, ref)
    alone = dec.decode_attention(store, q[4:5], table_d[4:5], lens_d[4:5], 256 ** -0.5, tier=bits, num_splits=1)
    assert torch.equal(alone[0], got[4])


@pytest.mark.parametrize("h,gqa,dt", [(8, 4, torch.float16), (3, 20, torch.bfloat16), (2, 4, torch.float32)])
@pytest.mark.parametrize("bits", [8, 4, 2])
def test_head_size_256_prefill_on_the_mfma_kernel(device, h, gqa, dt, bits):
    """Head size 256 prefill on the fused MFMA kernel (64 // GQA query tokens per
    tile, one 16-row block per wave): chunks of 1 to 300 tokens over contexts up to
    1000, GQA 4 and 20, fp16 / bf16 / float32 queries (the query lo part), odd KV
    head counts, K outlier channels x10 (cfg3's activations, as every prefill test
    here: prefill's V and P operands are single fp16 values); against the oracle."""
    lens = np.array([1, 17, 300, 64, 1000])
    store, table = build_layer(device, lens, bits, h=h, d=256, dtype=dt, seed=12, outliers=0.02)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    gen = torch.Generator(device=device)
    gen.manual_seed(120)
    prefill, row = [], 0
    for n in lens.tolist():
        nq = min(300, n)
        prefill.append((row, row + nq, n, 0))
        row += nq
    qp = torch.randn(row, gqa * h, 256, device=device, generator=gen).to(dt)
    out = torch.zeros(row, gqa * h, 256, device=device)
    pf.prefill_attention(store, qp, out, prefill, list(range(5)), table_d, 256 ** -0.5)
    torch.cuda.synchronize()
    ref = OA.prefill_attention(ps, qp.float().cpu().numpy(), prefill, list(range(5)), table, 256 ** -0.5,
                               vectorized=True)
    check(f"prefill D256 H{h} GQA{gqa} {str(dt)[6:]} int{bits}", out, ref)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_decode_over_a_layer_view_spanning_more_than_4_gib(device, bits):
    """One layer's view of a pool interleaved across 32 layers (page stride = 32
    pages): 4,000 blocks span about 5 GB, and the sequences' blocks sit above
    4 GiB while their pool chunks sit near the start. Decode must equal exact
    attention over the view's own gathered K/V (the gather kernel addresses
    pages with 64-bit arithmetic and is pinned to the oracle elsewhere)."""
    h, d, bs, kg, vg = 8, 128, 16, 16, 32
    page = bs * TieredLayout.per_token_bytes(h, d, 8, kg, vg)
    layers, nb = 32, 4000
    stride = page * layers
    assert nb * stride > 4 * 2 ** 30 + 2 ** 28
    backing = torch.zeros(nb * stride, dtype=torch.uint8, device=device)
    pages = torch.as_strided(backing, (nb, page), (stride, 1), storage_offset=5 * page)
    lens = np.array([700, 1500, 33, 2049])
    rng = np.random.default_rng(7)
    need = int((-(-(lens + 1) // bs)).sum())
    high = rng.permutation(np.arange(nb - 400, nb))[:need]
    table = np.zeros((len(lens), int((-(-(lens + 1) // bs)).max())), np.int64)
    o = 0
    for i, n in enumerate((-(-(lens + 1) // bs)).tolist()):
        table[i, :n] = high[o : o + n]
        o += n
    assert (table[table > 0] * stride > 4 * 2 ** 30).all()
    store, _ = build_layer(device, lens, bits, seed=7, pages=pages, table=table)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    gen = torch.Generator(device=device)
    gen.manual_seed(77)
    q = torch.randn(len(lens), 32, d, device=device, generator=gen).half()
    got = dec.decode_attention(store, q, table_d, torch.from_numpy(lens).to(device), d ** -0.5, tier=bits)
    ref = np.zeros(q.shape)
    for i, n in enumerate(lens.tolist()):
        pos = torch.arange(n, device=device)
        k, v = store.gather(table_d[i].long()[pos // bs], pos % bs)
        ref[i] = OA.attend(q[i].float().cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), d ** -0.5)
    check(f"> 4 GiB view int{bits}", got, ref)
    del backing


# ---- layers holding several tiers: tier passes -------------------------------------------

def build_mixed_layer(device, lens, cuts, tiers, *, h=8, d=128, bs=16, kg=16, vg=32, seed=5):
    """A layer written in len(tiers) steps: sequence i's tokens [cuts[j][i], cuts[j+1][i])
    at tiers[j] (block-aligned cuts, so each block keeps the tier it opened at, as
    after a controller's tier change). K carries 1% outlier channels x10."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int64)
    table, nb = block_table(rng, lens, bs)
    layout = TieredLayout(h, d, bs, 8, kg, vg)
    pages = torch.zeros(nb, bs * TieredLayout.per_token_bytes(h, d, 8, kg, vg), dtype=torch.uint8, device=device)
    store = TieredKVCache(layout, pages, residual_slots=len(lens) + 16, residual_dtype=torch.float16)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    out_ch = torch.randperm(h * d, generator=gen, device=device)[: round(0.01 * h * d)]
    for j, bits in enumerate(tiers):
        slots = slots_of(table, lens, lambda i, n: np.arange(cuts[j][i], cuts[j + 1][i]), bs)
        if not slots.size:
            continue
        k = torch.randn(slots.size, h, d, generator=gen, device=device)
        k.view(slots.size, h * d)[:, out_ch] *= 10
        v = torch.randn(slots.size, h, d, generator=gen, device=device)
        store.write(k.half(), v.half(), torch.from_numpy(slots).to(device), bits)
    torch.cuda.synchronize()
    return store, table


def test_mixed_tier_layer_with_tier_passes(device):
    """A layer holding INT4, INT8 and INT2 blocks (each context: first third INT4,
    second INT8, rest INT2; one context all INT8, one all INT4), decoded with one
    pipelined pass per tier (tier_mask), against the oracle: the mask read from the
    device, a mask naming an absent tier or missing a present one (the lowest pass
    takes the rest), a sequence alone equal bit for bit to itself in the batch, and a
    captured graph replayed under changing masks equal to eager calls."""
    rng = np.random.default_rng(31)
    lens = rng.integers(100, 3000, 24)
    c1, c2 = (lens // 3 // 16) * 16, (2 * lens // 3 // 16) * 16
    c1[0], c2[0] = 0, lens[0]  # all INT8
    c1[1] = c2[1] = lens[1]    # all INT4
    store, table = build_mixed_layer(device, lens, [np.zeros_like(lens), c1, c2, lens], [4, 8, 2])
    live = store.pool.live_tiers()
    print(f"[mixed] live blocks per tier {live}", flush=True)
    assert all(live[b] for b in (2, 4, 8))
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(32)
    q = torch.randn(len(lens), 32, 128, device=device, generator=gen).half()
    scale = 128 ** -0.5
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, scale, vectorized=True)
    ns = dec.default_splits(table_d, 16, 16, None)

    def run(mask, qq=q, tb=table_d, ln=lens_d, **kw):
        return dec.decode_attention(store, qq, tb, ln, scale, tier=4, tier_mask=mask, num_splits=ns, **kw)

    full = torch.tensor([2 | 4 | 8], dtype=torch.int32, device=device)
    got = run(full)
    check("mixed tiers, passes 2|4|8", got, ref)
    check("mixed tiers, passes from the pool", run("auto"), ref)
    for m in (4 | 8, 2 | 4, 8, 0):  # a present tier without a pass: the lowest pass's generic path
        check(f"mixed tiers, mask {m}", run(torch.tensor([m], dtype=torch.int32, device=device)), ref)
    check("mixed tiers, one pass (no mask)", run(None), ref)
    for i in (0, 1, 5):
        alone = run(full, q[i : i + 1], table_d[i : i + 1], lens_d[i : i + 1])
        assert torch.equal(alone[0], got[i]), f"sequence {i}: alone differs from in the batch"

    mask = full.clone()
    out = torch.empty_like(got)
    rows = dec.workspace_rows(store, 32, q.dtype, len(lens), ns, _lib.DECODE_BATCH_INVARIANT)
    ws = (torch.empty(rows, 32, 128, device=device), torch.empty(rows, 32, 2, device=device))
    run(mask, out=out, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(mask, out=out, workspace=ws)
    for m in (2 | 4 | 8, 4 | 8, 4, 0, 2 | 4 | 8):
        mask.fill_(m)
        graph.replay()
        torch.cuda.synchronize()
        eager = run(torch.tensor([m], dtype=torch.int32, device=device))
        assert torch.equal(out, eager), f"graph replay with mask {m} differs from the eager call"
        check(f"mixed tiers, graph replay, mask {m}", out, ref)


@pytest.mark.parametrize("d,gqa,qdt,ws", [(64, 4, torch.float16, None), (128, 4, torch.float32, None),
                                          (128, 20, torch.float16, None), (128, 4, torch.float16, "static"),
                                          (256, 4, torch.float16, None), (256, 4, torch.float32, None)])
def test_tier_passes_at_other_shapes(device, d, gqa, qdt, ws):
    """Tier passes at head sizes 64 and 256 (half-heads), with float32 queries (the
    query hi / lo path), at GQA 20 (query heads in groups of 16, each group its own
    passes) and on the library's static workspace: against the oracle, and equal to
    themselves when a sequence is decoded alone."""
    h = 4
    rng = np.random.default_rng(40 + d + gqa)
    lens = rng.integers(60, 1500, 12)
    c1, c2 = (lens // 3 // 16) * 16, (2 * lens // 3 // 16) * 16
    store, table = build_mixed_layer(device, lens, [np.zeros_like(lens), c1, c2, lens], [8, 2, 4], h=h, d=d, seed=41)
    ps = oracle_view(store)
    table_d = torch.from_numpy(table).to(device, torch.int32)
    lens_d = torch.from_numpy(lens).to(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(42)
    q = torch.randn(len(lens), h * gqa, d, device=device, generator=gen).to(qdt)
    ref = OA.decode_attention(ps, q.float().cpu().numpy(), table, lens, d ** -0.5, vectorized=True)
    mask = torch.tensor([2 | 4 | 8], dtype=torch.int32, device=device)
    ns = dec.default_splits(table_d, 16, 16, None)
    kw = dict(tier=4, tier_mask=mask, num_splits=ns, workspace=ws)
    got = dec.decode_attention(store, q, table_d, lens_d, d ** -0.5, **kw)
    check(f"tier passes D{d} GQA{gqa} {str(qdt)[6:]}{' static' if ws else ''}", got, ref)
    alone = dec.decode_attention(store, q[3:4], table_d[3:4], lens_d[3:4], d ** -0.5, **kw)
    assert torch.equal(alone[0], got[3])
