"""GPU: echokv_decode_static (no workspace arguments; acc / ml in the library's
static device scratch) against echokv_decode with caller-owned workspaces, bit
for bit, on two calls in a row (the second smaller), inside a captured HIP graph,
and its refusal of a request larger than the scratch."""

import numpy as np
import pytest
import torch

import scripts as S
from echokv_amd.kernels import decode as dec
from gpu_util import gpu_replay, t

pytestmark = pytest.mark.gpu


def _inputs(device, case, hq_per_kv, seed):
    s = S.decode_case(case)
    store, *_ = gpu_replay(s, device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    n = len(s.meta["lens"])
    q = torch.randn(n, hq_per_kv * s.h, s.d, device=device, generator=gen).half()
    table = t(s.meta["table"], device, torch.int32)
    lens = t(s.meta["lens"], device).long()
    return s, store, q, table, lens


def _pair(store, q, table, lens, s, splits):
    """(echokv_decode output, echokv_decode_static output) on the same inputs."""
    ref = torch.empty(q.shape, device=q.device)
    got = torch.full(q.shape, 5.0, device=q.device)
    dec.decode_attention(store, q, table, lens, s.d ** -0.5, blocks_per_split=2, num_splits=splits, out=ref)
    dec.decode_attention(store, q, table, lens, s.d ** -0.5, blocks_per_split=2, num_splits=splits, out=got,
                         workspace="static")
    torch.cuda.synchronize()
    return ref, got


def test_static_decode_equals_workspace_decode_on_consecutive_calls(device):
    s4, st4, q4, tb4, ln4 = _inputs(device, 4, 4, 1)   # larger call first
    s1, st1, q1, tb1, ln1 = _inputs(device, 1, 2, 2)   # then a smaller one
    before = torch.cuda.memory_allocated()
    ref, got = _pair(st4, q4, tb4, ln4, s4, 8)
    print(f"[static decode] call 1: {tuple(q4.shape)}, 8 splits", flush=True)
    assert torch.equal(ref, got)
    ref1, got1 = _pair(st1, q1, tb1, ln1, s1, 3)
    print(f"[static decode] call 2: {tuple(q1.shape)}, 3 splits", flush=True)
    assert torch.equal(ref1, got1)
    assert torch.isfinite(got1).all()
    # The static calls allocate nothing through torch (both outputs were preallocated).
    ref2 = torch.empty_like(q1, dtype=torch.float32)
    dec.decode_attention(st1, q1, tb1, ln1, s1.d ** -0.5, blocks_per_split=2, num_splits=3, out=ref2)
    torch.cuda.synchronize()
    mid = torch.cuda.memory_allocated()
    dec.decode_attention(st1, q1, tb1, ln1, s1.d ** -0.5, blocks_per_split=2, num_splits=3, out=ref2,
                         workspace="static")
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == mid
    assert mid >= before


def test_static_decode_replays_in_a_captured_graph(device):
    s, store, q, table, lens = _inputs(device, 4, 4, 3)
    out = torch.zeros(q.shape, device=device)
    static_q = q.clone()
    dec.decode_attention(store, static_q, table, lens, s.d ** -0.5, blocks_per_split=2, num_splits=4, out=out,
                         workspace="static")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dec.decode_attention(store, static_q, table, lens, s.d ** -0.5, blocks_per_split=2, num_splits=4, out=out,
                             workspace="static")
    for rep in range(3):
        static_q.copy_(torch.randn(q.shape, device=device).half())
        g.replay()
        torch.cuda.synchronize()
        ref = torch.empty_like(out)
        dec.decode_attention(store, static_q, table, lens, s.d ** -0.5, blocks_per_split=2, num_splits=4, out=ref)
        torch.cuda.synchronize()
        print(f"[static decode] graph replay {rep}", flush=True)
        assert torch.equal(out, ref)


def test_static_decode_refuses_requests_beyond_the_scratch(device):
    s, store, q, table, lens = _inputs(device, 1, 2, 4)
    big = 64 * 2 ** 20 // ((s.d + 2) * 4 * q.shape[1] * len(lens)) + 1  # splits that overflow 64 MiB
    out = torch.zeros(q.shape, device=device)
    with pytest.raises(RuntimeError, match="static scratch"):
        dec.decode_attention(store, q, table, lens, s.d ** -0.5, num_splits=big, out=out, workspace="static")
    assert (out == 0).all()
    np.testing.assert_array_equal(out.cpu().numpy(), 0)
