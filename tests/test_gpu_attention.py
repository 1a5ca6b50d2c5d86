"""GPU: decode (split-KV MFMA + merge) and chunked prefill (MFMA) against the
float64 oracle and the reference's own outputs, at the north-star tolerance
(2e-3 max-abs; for fp16 / bf16 outputs, beyond the output's own rounding); plus the reference decode tests' batch-invariance, indexed
rows, never-opened blocks and graph-padding properties
(tests/echokv_vllm/test_decode_kernel.py:88-190, test_prefill_kernel.py)."""

import numpy as np
import pytest
import torch

import scripts as S
from echokv_amd.kernels import decode as dec
from echokv_amd.kernels import prefill as pf
from gpu_util import gpu_replay, maxdiff, t
from host_sim import golden, replay
from oracle import attention as OA

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module")
def case_stores(device):
    out = {}
    for i in range(len(S.DECODE_CASES)):
        s = S.decode_case(i)
        sim = replay(s)
        store, *_ = gpu_replay(s, device)
        out[i] = (s, sim, store)
    return out


@pytest.mark.parametrize("name", ["cfg1_int8_bs16", "cfg1_int4_bs16", "cfg1_int2_bs16", "cfg1_int4_bs32"])
def test_cfg1_decode_matches_reference_output(device, name):
    print(f"[decode] {name}", flush=True)
    s = next(x for x in S.all_scripts() if x.name == name)
    g = golden(name)
    store, *_ = gpu_replay(s, device)
    q = S.cfg1_query(s)
    table = t(s.meta["table"], device, torch.int32)
    lens = t(s.meta["lens"], device)
    for bps in (1, 4, 16):
        for inv in (False, True):
            got = dec.decode_attention(store, t(q, device), table, lens, s.d ** -0.5, blocks_per_split=bps,
                                       batch_invariant=inv)
            torch.cuda.synchronize()
            err = maxdiff(got, g["decode_out"])
            assert err <= TOL, f"{name} bps={bps} invariant={inv}: max err {err}"


@pytest.mark.parametrize("i", range(len(S.DECODE_CASES)))
@pytest.mark.parametrize("bps", [1, 3])
@pytest.mark.parametrize("qdt", [torch.float16, torch.float32])
@pytest.mark.parametrize("inv", [False, True], ids=["balanced", "split"])
def test_decode_matches_oracle(device, case_stores, i, bps, qdt, inv):
    s, sim, store = case_stores[i]
    print(f"[decode] {s.name} bps={bps} {qdt}", flush=True)
    table = t(s.meta["table"], device, torch.int32)
    lens = t(s.meta["lens"], device)
    for gqa in (1, 4, 7):
        rng = np.random.default_rng(100 + gqa)
        q = rng.standard_normal((len(s.meta["lens"]), gqa * s.h, s.d), dtype=np.float32)
        qt = t(q, device, qdt)
        ref = OA.decode_attention(sim.ps, qt.float().cpu().numpy(), s.meta["table"], s.meta["lens"], s.d ** -0.5)
        got = dec.decode_attention(store, qt, table, lens, s.d ** -0.5, blocks_per_split=bps, batch_invariant=inv)
        torch.cuda.synchronize()
        err = maxdiff(got, ref)
        assert err <= TOL, f"{s.name} gqa={gqa} bps={bps}: max err {err}"


@pytest.mark.parametrize("gqa", [17, 32])
@pytest.mark.parametrize("inv", [False, True], ids=["balanced", "split"])
def test_decode_gqa_above_16_matches_oracle(device, case_stores, gqa, inv):
    """GQA beyond one MFMA column block (16 query heads per KV head) runs in passes
    of 16 query heads; every query head's row against the oracle."""
    for i in (0, 3):
        s, sim, store = case_stores[i]
        print(f"[decode] {s.name} gqa={gqa}", flush=True)
        table = t(s.meta["table"], device, torch.int32)
        lens = t(s.meta["lens"], device)
        rng = np.random.default_rng(gqa)
        q = rng.standard_normal((len(s.meta["lens"]), gqa * s.h, s.d), dtype=np.float32)
        qt = t(q, device, torch.float16)
        ref = OA.decode_attention(sim.ps, qt.float().cpu().numpy(), s.meta["table"], s.meta["lens"], s.d ** -0.5)
        got = dec.decode_attention(store, qt, table, lens, s.d ** -0.5, blocks_per_split=2, batch_invariant=inv)
        torch.cuda.synchronize()
        err = maxdiff(got, ref)
        assert err <= TOL, f"{s.name} gqa={gqa}: max err {err}"


@pytest.mark.parametrize("scale", [-0.088, 0.0, 0.9])
def test_decode_softmax_scale_sign_and_zero(device, case_stores, scale):
    """The kernels take the max on unscaled scores and scale inside the
    exponent; a negative scale (query sign flipped) and a zero one (every
    weight equal) must still match the oracle's softmax(scale * q.k)."""
    for i in range(len(S.DECODE_CASES)):
        s, sim, store = case_stores[i]
        print(f"[decode] {s.name} scale={scale}", flush=True)
        table = t(s.meta["table"], device, torch.int32)
        lens = t(s.meta["lens"], device)
        rng = np.random.default_rng(7)
        q = rng.standard_normal((len(s.meta["lens"]), 4 * s.h, s.d), dtype=np.float32)
        qt = t(q, device, torch.float16)
        ref = OA.decode_attention(sim.ps, qt.float().cpu().numpy(), s.meta["table"], s.meta["lens"], scale)
        for inv in (False, True):
            got = dec.decode_attention(store, qt, table, lens, scale, blocks_per_split=2, batch_invariant=inv)
            torch.cuda.synchronize()
            err = maxdiff(got, ref)
            assert err <= TOL, f"{s.name} scale={scale} invariant={inv}: max err {err}"


def test_decode_is_batch_invariant(device, case_stores):
    s, sim, store = case_stores[0]
    table = t(s.meta["table"], device, torch.int32)
    lens = t(s.meta["lens"], device)
    q = torch.randn(len(s.meta["lens"]), 2 * s.h, s.d, device=device)
    full = dec.decode_attention(store, q, table, lens, s.d ** -0.5, 2, batch_invariant=True)
    for i in range(len(s.meta["lens"])):
        nb = -(-int(s.meta["lens"][i]) // s.bs)
        alone = dec.decode_attention(store, q[i : i + 1], table[i : i + 1, :nb], lens[i : i + 1], s.d ** -0.5, 2,
                                     batch_invariant=True)
        assert torch.equal(alone[0], full[i])


def test_decode_indexed_rows_into_bf16_output(device, case_stores):
    s, sim, store = case_stores[0]
    table = t(s.meta["table"], device, torch.int32)
    lens = t(s.meta["lens"], device)
    hq = 2 * s.h
    q_all = torch.randn(7, hq, s.d, device=device)
    q_rows = torch.tensor([6, 1, 3], device=device)
    bt_rows = torch.tensor([4, 0, 2], device=device)
    sel = lens[bt_rows]
    out = torch.full((7, hq, s.d), 7.0, device=device, dtype=torch.bfloat16)
    dec.decode_attention(store, q_all, table, sel, s.d ** -0.5, 2, q_rows=q_rows, bt_rows=bt_rows, out=out,
                         max_len=int(sel.max()), batch_invariant=True)
    ref = OA.decode_attention(sim.ps, q_all[q_rows].cpu().numpy(), s.meta["table"][[4, 0, 2]],
                              s.meta["lens"][[4, 0, 2]], s.d ** -0.5)
    assert maxdiff(out[q_rows], ref) <= 2e-2  # bf16 output rounding
    untouched = [r for r in range(7) if r not in q_rows.tolist()]
    assert (out[untouched] == 7.0).all()
    wide = torch.zeros_like(out)  # a wider split grid must not change any bit (split schedule)
    dec.decode_attention(store, q_all, table, sel, s.d ** -0.5, 2, q_rows=q_rows, bt_rows=bt_rows, out=wide,
                         batch_invariant=True)
    assert torch.equal(wide[q_rows], out[q_rows])


def test_never_opened_blocks_are_safe(device, case_stores):
    s, sim, store = case_stores[0]
    used = set(s.meta["table"][s.meta["table"] >= 0].ravel().tolist())
    unused = [b for b in range(s.num_blocks) if b not in used and int(store.tag[b]) == 0][:2]
    assert len(unused) == 2
    fresh = torch.tensor([unused], dtype=torch.int32, device=device)
    q = torch.randn(1, 2 * s.h, s.d, device=device)
    out = dec.decode_attention(store, q, fresh, torch.tensor([100], device=device), s.d ** -0.5, 4)
    assert torch.isfinite(out).all()
    b = unused[0]
    k = torch.randn(3, s.h, s.d, device=device)
    store.write(k, k, b * s.bs + 5 + torch.arange(3, device=device), 4)
    assert int(store.tag[b]) == 4


def test_graph_padding_and_fixed_split_grid(device, case_stores):
    s, sim, store = case_stores[2]  # 500 tokens and 3 tokens
    table = t(s.meta["table"], device, torch.int32)
    hq = 2 * s.h
    q_all = torch.randn(4, hq, s.d, device=device)
    q_rows = torch.arange(4, device=device)
    bt_rows = torch.tensor([0, 1, 0, 0], device=device)
    sel = torch.tensor([500, 3, 0, 0], device=device)
    out = torch.full((4, hq, s.d), 7.0, device=device, dtype=torch.bfloat16)
    dec.decode_attention(store, q_all, table, sel, s.d ** -0.5, 2, q_rows=q_rows, bt_rows=bt_rows, out=out,
                         num_splits=3, batch_invariant=True)
    ref = OA.decode_attention(sim.ps, q_all[:2].cpu().numpy(), s.meta["table"], s.meta["lens"], s.d ** -0.5)
    assert maxdiff(out[:2], ref) <= 2e-2
    assert (out[2:] == 7.0).all()
    alone = torch.zeros_like(out[:1])
    dec.decode_attention(store, q_all[:1], table[:1], torch.tensor([500], device=device), s.d ** -0.5, 2, out=alone,
                         num_splits=3, batch_invariant=True)
    assert torch.equal(alone[0], out[0])


# ---- prefill -------------------------------------------------------------------------

PATHS = {"fused": pf.prefill_attention_fused, "dense": pf.prefill_attention_dense}


@pytest.mark.parametrize("path", sorted(PATHS))
def test_cfg1_prefill_matches_reference_output(device, path):
    s = next(x for x in S.all_scripts() if x.name == "cfg1_int4_bs16")
    g = golden(s.name)
    store, *_ = gpu_replay(s, device)
    prefill, req_of, q = S.cfg1_prefill(s)
    table = t(s.meta["table"], device, torch.int32)
    for qdt in (torch.float32, torch.float16, torch.bfloat16):
        print(f"[prefill cfg1] {path} {qdt}", flush=True)
        qt = t(q, device, qdt)
        out = torch.zeros(q.shape, device=device, dtype=torch.float32)
        PATHS[path](store, qt, out, prefill, req_of, table, s.d ** -0.5)
        torch.cuda.synchronize()
        if qdt == torch.float32:
            err = maxdiff(out, g["prefill_out"])
        else:  # the oracle on the same rounded queries
            from host_sim import replay as rp

            sim = rp(s)
            err = maxdiff(out, OA.prefill_attention(sim.ps, qt.float().cpu().numpy(), prefill, req_of,
                                                    s.meta["table"], s.d ** -0.5))
        assert err <= TOL, f"{qdt}: max err {err}"


@pytest.mark.parametrize("chunk", [200, 1000])
def test_cfg1_long_chunk_prefill_matches_oracle(device, chunk):
    """Long chunks (the two-pass path): each sequence's last ``chunk`` tokens (or
    all of them) over its whole context, several query and key tiles per request."""
    s = next(x for x in S.all_scripts() if x.name == "cfg1_int4_bs16")
    sim = replay(s)
    store, *_ = gpu_replay(s, device)
    prefill, req_of, row = [], [], 0
    for r, n in enumerate(S.CFG1_LENS):
        nq = min(chunk, n)
        prefill.append((row, row + nq, n, 0))
        req_of.append(r)
        row += nq
    q = np.random.default_rng(chunk).standard_normal((row, 32, s.d), dtype=np.float32)
    qt = t(q, device, torch.bfloat16)
    out = torch.zeros(q.shape, device=device, dtype=torch.float32)
    print(f"[prefill long] chunk={chunk}", flush=True)
    pf.prefill_attention(store, qt, out, prefill, req_of, t(s.meta["table"], device, torch.int32), s.d ** -0.5)
    torch.cuda.synchronize()
    assert pf.use_dense(prefill, s.d)
    ref = OA.prefill_attention(sim.ps, qt.float().cpu().numpy(), prefill, req_of, s.meta["table"], s.d ** -0.5)
    err = maxdiff(out, ref)
    assert err <= TOL, f"chunk {chunk}: max err {err}"


PREFILL_CASES = [  # decode case index, ctx == its lens, chunk lengths
    (0, [1, 40, 64, 65, 200], [1, 40, 1, 65, 77]),
    (3, [200, 70], [17, 70]),
    (1, [33, 97, 128], [33, 50, 128]),
    (4, [300, 17, 1, 129], [300, 16, 1, 100]),
]


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("case", PREFILL_CASES)
@pytest.mark.parametrize("gqa", [1, 4, 7])
def test_prefill_matches_oracle(device, case_stores, case, gqa, path):
    i, ctxs, chunks = case
    s, sim, store = case_stores[i]
    print(f"[prefill] {path} {s.name} gqa={gqa}", flush=True)
    prefill, req_of, row = [], [], 0
    for r, (ctx, nq) in enumerate(zip(ctxs, chunks)):
        prefill.append((row, row + nq, ctx, 0))
        req_of.append(r)
        row += nq
    q = np.random.default_rng(gqa).standard_normal((row, gqa * s.h, s.d), dtype=np.float32)
    qt = t(q, device, torch.float16)
    out = torch.zeros(row, gqa * s.h, s.d, device=device)
    PATHS[path](store, qt, out, prefill, req_of, t(s.meta["table"], device, torch.int32), s.d ** -0.5)
    torch.cuda.synchronize()
    ref = OA.prefill_attention(sim.ps, qt.float().cpu().numpy(), prefill, req_of, s.meta["table"], s.d ** -0.5)
    err = maxdiff(out, ref)
    assert err <= TOL, f"{s.name} gqa={gqa}: max err {err}"


@pytest.mark.parametrize("i", [0, 1, 4])
def test_dequant_dense_matches_gather(device, case_stores, i):
    s, sim, store = case_stores[i]
    lens = s.meta["lens"].tolist()
    prefill, starts, g = [], [], 0
    for ctx in lens:
        starts.append(g)
        prefill.append((0, 1, ctx, g))
        g += ctx
    work = pf.build_dequant_work(prefill, list(range(len(lens))), s.bs, device)
    k, v = pf.dequant_dense(store, work, g, t(s.meta["table"], device, torch.int32), torch.float32)
    torch.cuda.synchronize()
    for r, (ctx, st) in enumerate(zip(lens, starts)):
        kr, vr = sim.ps.gather_seq(s.meta["table"][r], ctx)
        np.testing.assert_array_equal(k[st : st + ctx].cpu().numpy(), kr)
        np.testing.assert_array_equal(v[st : st + ctx].cpu().numpy(), vr)
