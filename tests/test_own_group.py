"""Own-group-exact prefill (the fix ``echokv_vllm`` docs/ECHOKV_VLLM_PLUGIN.md:261-266
names for preempted / re-chunked requests). The property that defines it: a
request prefilled again -- in one chunk, or in chunks that start on K-group
boundaries, as prefix caching and group-multiple chunk budgets give -- attends
exactly as decode did when each token was the newest (its own group then open,
read at full precision from the residual). CPU: the oracle has that property,
against the oracle decode on a store written token by token; GPU: the kernels
(both prefill paths) against the oracle and against the decode kernel's own
decode-time outputs, within 2e-3."""

import numpy as np
import pytest
import torch

import scripts as S
from host_sim import SimStore
from oracle import attention as OA

H, D, BS, KG, HQ, N = 2, 64, 16, 16, 8, 100


def script(chunks, seed=4):
    """One sequence of N tokens written in the given chunks (INT4 blocks)."""
    nb = -(-N // BS) + 2
    table = np.random.default_rng(seed).permutation(nb)[: -(-N // BS)]
    steps, p = [], 0
    for c in chunks:
        pos = np.arange(p, p + c)
        steps.append((table[pos // BS] * BS + pos % BS, 4))
        p += c
    assert p == N
    s = S.Script("own_group", H, D, BS, 8, KG, 32, nb, 4, steps, seed=seed, dtype="f16", full_bytes=False)
    s.meta = {"table": table[None, :], "lens": np.array([N])}
    return s


def inputs():
    """K / V rows of the N tokens (K channel 1 carries a +30 outlier) and one query per token."""
    rng = np.random.default_rng(8)
    k = rng.standard_normal((N, H, D)).astype(np.float32)
    k[..., 1] += 30.0
    v = rng.standard_normal((N, H, D)).astype(np.float32)
    q = rng.standard_normal((N, HQ, D)).astype(np.float32)
    return k.astype(np.float16), v.astype(np.float16), q.astype(np.float16)


def steps(s, k, v):
    """(slots, bits, K rows, V rows) of each of the script's chunks."""
    p0 = 0
    for slots, bits in s.steps:
        yield slots, bits, k[p0 : p0 + slots.size], v[p0 : p0 + slots.size]
        p0 += slots.size


def decode_time_outputs():
    """Oracle decode of token p right after it was written (its group open)."""
    s = script([1] * N)
    k, v, q = inputs()
    sim = SimStore(s)
    out = np.zeros((N, HQ, D))
    for p, (slots, bits, kk, vv) in enumerate(steps(s, k, v)):
        sim.write(kk, vv, slots, bits)
        out[p] = OA.decode_attention(sim.ps, q[p : p + 1].astype(np.float32), s.meta["table"], [p + 1],
                                     D ** -0.5, vectorized=True)[0]
    return out, k, v, q


@pytest.fixture(scope="module")
def decode_time():
    return decode_time_outputs()


@pytest.mark.parametrize("chunks", [[N], [48, 52], [16, 32, 16, 36]], ids=["one", "48+52", "16+32+16+36"])
def test_oracle_own_group_prefill_equals_decode_time_attention(decode_time, chunks):
    ref, k, v, q = decode_time
    s = script(chunks)
    sim = SimStore(s)
    p0 = 0
    for (slots, bits, kk, vv), c in zip(steps(s, k, v), chunks):
        sim.write(kk, vv, slots, bits)
        got = OA.prefill_own_group_exact(sim.ps, q[p0 : p0 + c].astype(np.float32), kk.astype(np.float32),
                                         [(0, c, p0 + c, 0)], [0], s.meta["table"], D ** -0.5)
        assert np.abs(got - ref[p0 : p0 + c]).max() < 1e-9, f"chunk at {p0}"
        p0 += c


def test_oracle_own_group_differs_from_plain_prefill_only_inside_groups(decode_time):
    """Plain prefill reads every query's own group back quantized once the group is
    complete; own-group-exact prefill differs from it there, and agrees where the
    group is still open in the store (the last, partial group: exact in both)."""
    ref, k, v, q = decode_time
    s = script([N])
    sim = SimStore(s)
    for slots, bits, kk, vv in steps(s, k, v):
        sim.write(kk, vv, slots, bits)
    plain = OA.prefill_attention(sim.ps, q.astype(np.float32), [(0, N, N, 0)], [0], s.meta["table"], D ** -0.5,
                                 vectorized=True)
    og = OA.prefill_own_group_exact(sim.ps, q.astype(np.float32), k.astype(np.float32), [(0, N, N, 0)], [0],
                                    s.meta["table"], D ** -0.5)
    diff = np.abs(plain - og).max(axis=(1, 2))
    closed = np.arange(N) < (N // KG) * KG  # groups complete (quantized) in the final store
    assert diff[closed].max() > 1e-4  # the quantization error of the own group shows
    assert diff[~closed].max() < 1e-9  # the open last group is read exactly by both


# ---- GPU -----------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("chunks", [[N], [48, 52], [16, 32, 16, 36]], ids=["dense", "fused", "fused-4"])
def test_hip_own_group_prefill_matches_oracle_and_decode_time(device, decode_time, chunks):
    """Both prefill paths with own-group-exact on: each chunk, right after it is
    written, against the oracle over the same pages and against decode-time
    attention (the oracle decode when each token was the newest), within 2e-3."""
    from echokv_amd.kernels import prefill as pf
    from gpu_util import gpu_store, maxdiff
    from oracle import store as OS

    ref, k, v, q = decode_time
    s = script(chunks)
    store, *_ = gpu_store(s, device)
    table = torch.from_numpy(s.meta["table"]).to(device, torch.int32)
    p0, worst_o, worst_d = 0, 0.0, 0.0
    for (slots, bits, kk, vv), c in zip(steps(s, k, v), chunks):
        kt, vt = torch.from_numpy(kk).to(device), torch.from_numpy(vv).to(device)
        store.write(kt, vt, torch.from_numpy(slots).to(device), bits)
        qt = torch.from_numpy(q[p0 : p0 + c]).to(device)
        out = torch.zeros(c, HQ, D, device=device, dtype=torch.float32)
        prefill = [(0, c, p0 + c, 0)]
        pf.prefill_attention(store, qt, out, prefill, [0], table, D ** -0.5, own_group_key=kt)
        torch.cuda.synchronize()
        L = store.layout
        ps = OS.PageStore.over(OS.Layout(L.num_kv_heads, L.head_size, L.block_size, L.mem_bits, L.k_group, L.v_group),
                               store.pages.cpu().numpy(), store.res_k.float().cpu().numpy(),
                               store.block_res.cpu().numpy(), store.res_group.cpu().numpy())
        oracle = OA.prefill_own_group_exact(ps, q[p0 : p0 + c].astype(np.float32), kk.astype(np.float32), prefill,
                                            [0], s.meta["table"], D ** -0.5)
        worst_o = max(worst_o, maxdiff(out, oracle))
        worst_d = max(worst_d, maxdiff(out, ref[p0 : p0 + c]))
        p0 += c
    print(f"[own-group {chunks}] vs oracle {worst_o:.3e}, vs decode-time {worst_d:.3e}", flush=True)
    assert worst_o <= 2e-3 and worst_d <= 2e-3


@pytest.mark.gpu
def test_hip_own_group_off_leaves_prefill_unchanged(device, decode_time):
    """Without a key the prefill kernels run as before (no own-group mask)."""
    from echokv_amd.kernels import prefill as pf
    from gpu_util import gpu_store, maxdiff
    from oracle import store as OS

    ref, k, v, q = decode_time
    s = script([N])
    store, *_ = gpu_store(s, device)
    for slots, bits, kk, vv in steps(s, k, v):
        store.write(torch.from_numpy(kk).to(device), torch.from_numpy(vv).to(device),
                    torch.from_numpy(slots).to(device), bits)
    table = torch.from_numpy(s.meta["table"]).to(device, torch.int32)
    out = torch.zeros(N, HQ, D, device=device)
    pf.prefill_attention(store, torch.from_numpy(q).to(device), out, [(0, N, N, 0)], [0], table, D ** -0.5)
    torch.cuda.synchronize()
    L = store.layout
    ps = OS.PageStore.over(OS.Layout(L.num_kv_heads, L.head_size, L.block_size, L.mem_bits, L.k_group, L.v_group),
                           store.pages.cpu().numpy(), store.res_k.float().cpu().numpy(),
                           store.block_res.cpu().numpy(), store.res_group.cpu().numpy())
    plain = OA.prefill_attention(ps, q.astype(np.float32), [(0, N, N, 0)], [0], s.meta["table"], D ** -0.5,
                                 vectorized=True)
    assert maxdiff(out, plain) <= 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize("own_group", [False, True], ids=["plain", "own-group"])
def test_hip_prefix_cached_request_reads_the_shared_blocks(device, decode_time, own_group):
    """Prefix caching: request B's block table starts with request A's three blocks
    (48 tokens, written by A); B writes only its own tokens 48..99 into fresh
    blocks, then prefills that chunk over the whole context. Its attention equals
    the oracle's over the same pages, and equals what B gets had it written the
    whole sequence itself (the shared prefix holds the same bytes)."""
    from echokv_amd.kernels import prefill as pf
    from gpu_util import gpu_store, maxdiff
    from oracle import store as OS

    ref, k, v, q = decode_time
    nb = -(-N // BS)
    s = script([48, N - 48])
    s.num_blocks = 2 * nb + 2
    store, *_ = gpu_store(s, device)
    table_a = np.arange(nb)
    table_b = np.concatenate([table_a[:3], nb + np.arange(nb - 3)])  # shares A's first three blocks
    pos = np.arange(48)
    store.write(torch.from_numpy(k[:48]).to(device), torch.from_numpy(v[:48]).to(device),
                torch.from_numpy(table_a[pos // BS] * BS + pos % BS).to(device), 4)
    pos = np.arange(48, N)
    kb = torch.from_numpy(k[48:]).to(device)
    store.write(kb, torch.from_numpy(v[48:]).to(device), torch.from_numpy(table_b[pos // BS] * BS + pos % BS).to(device),
                4)
    table = torch.from_numpy(np.stack([table_a, table_b])).to(device, torch.int32)
    out = torch.zeros(N - 48, HQ, D, device=device)
    prefill = [(0, N - 48, N, 0)]
    pf.prefill_attention(store, torch.from_numpy(q[48:]).to(device), out, prefill, [1], table, D ** -0.5,
                         own_group_key=kb if own_group else None)
    torch.cuda.synchronize()
    L = store.layout
    ps = OS.PageStore.over(OS.Layout(L.num_kv_heads, L.head_size, L.block_size, L.mem_bits, L.k_group, L.v_group),
                           store.pages.cpu().numpy(), store.res_k.float().cpu().numpy(),
                           store.block_res.cpu().numpy(), store.res_group.cpu().numpy())
    tb = np.stack([table_a, table_b])
    if own_group:
        oracle = OA.prefill_own_group_exact(ps, q[48:].astype(np.float32), k[48:].astype(np.float32), prefill, [1],
                                            tb, D ** -0.5)
        assert maxdiff(out, ref[48:]) <= 2e-3  # and what decode saw, token by token
    else:
        oracle = OA.prefill_attention(ps, q[48:].astype(np.float32), prefill, [1], tb, D ** -0.5, vectorized=True)
    assert maxdiff(out, oracle) <= 2e-3
