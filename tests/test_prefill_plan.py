"""Host-side tile tables of chunked prefill: the fused kernel's query tiles and
the two-pass path's workspace and query tiles cover every query row and every
context key exactly once (echokv_vllm/kernels/prefill.py:56-87)."""

from echokv_amd.kernels import prefill as pf


def test_tiles_cover_every_query_row():
    prefill = [(0, 70, 70, 0), (70, 110, 200, 0), (110, 111, 33, 0)]
    for gqa in (1, 4, 7):
        tiles = pf.build_tiles(prefill, [0, 1, 2], gqa, "cpu")
        covered = sorted(r for q0, n, *_ in tiles.tolist() for r in range(q0, q0 + n))
        assert covered == list(range(111))
        assert all(n <= pf.block_m(gqa) for _, n, *_ in tiles.tolist())
        assert tiles[0].tolist()[2] == 0 and any(x[2] == 160 for x in tiles.tolist())


def test_dense_plan_covers_rows_and_contexts():
    prefill = [(0, 70, 70, 0), (70, 110, 200, 0), (110, 111, 33, 0), (111, 611, 900, 0)]
    for gqa in (1, 4, 7):
        plan = pf.build_dense_plan(prefill, [0, 1, 2, 5], gqa, "cpu")
        qt, packs = plan.qtiles.tolist(), plan.packs.tolist()
        covered = sorted(r for q0, n, *_ in qt for r in range(q0, q0 + n))
        assert covered == list(range(611))
        assert all(0 < n <= pf.dense_block_m(gqa) for _, n, *_ in qt)
        for q0, n, pos0, ctx, t0 in qt:
            (qs, qe, c, _), r = next((p, r) for p, r in zip(prefill, [0, 1, 2, 5]) if p[0] <= q0 < p[1])
            assert ctx == c and pos0 == c - (qe - qs) + (q0 - qs)
            keys = [k0 for rr, k0, cc in packs[t0 : t0 + -(-c // pf.DENSE_KEYS)]]
            assert keys == list(range(0, c, pf.DENSE_KEYS))
            assert all(rr == r and cc == c for rr, _, cc in packs[t0 : t0 + len(keys)])
        # heaviest request first
        assert qt[0][3] == 900


def test_fused_prefill_refuses_tiles_larger_than_its_kernel_takes():
    """Tiles built for the MFMA kernel (block_m tokens) handed to a layout that
    takes the fp32 kernel (any_block_m tokens) are refused on the host, tagged
    or not, before any device work; tiles of the right size pass the check."""
    import pytest
    import torch
    from types import SimpleNamespace

    store = SimpleNamespace(layout=SimpleNamespace(num_kv_heads=2, head_size=80), pages=torch.zeros(1))
    gqa = 4
    q = torch.zeros(40, 2 * gqa, 80)
    prefill, req = [(0, 40, 40, 0)], [0]
    assert not pf.kernels_take(80, gqa) and pf.block_m(gqa) > pf.any_block_m(gqa)
    big = pf.build_tiles(prefill, req, gqa, "cpu")
    for tiles in (big, big.clone()):  # tagged by build_tiles, and an untagged copy
        with pytest.raises(ValueError, match="at most"):
            pf.prefill_attention_fused(store, q, q, prefill, req, torch.zeros(1, 1), 0.1, tiles)
    ok = pf.build_tiles(prefill, req, gqa, "cpu", tokens=pf.any_block_m(gqa))
    with pytest.raises(RuntimeError, match="device tensors"):  # past the check: CPU tensors are refused next
        pf.prefill_attention_fused(store, q, q, prefill, req, torch.zeros(1, 1), 0.1, ok)


def test_head_size_256_tiles_hold_half_the_rows():
    """At head size 256 the fused MFMA kernel takes 64 query rows per tile (64 //
    GQA tokens): tiles built at head size 128's size are refused on the host,
    tiles of the right size pass; own-group-exact prefill is not offered there."""
    import pytest
    import torch
    from types import SimpleNamespace

    gqa = 4
    assert pf.kernels_take(256, gqa) and not pf.own_group_takes(256, gqa) and pf.own_group_takes(128, gqa)
    assert pf.block_m(gqa, 256) == 16 and pf.block_m(gqa) == 32 and not pf.kernels_take(256, 80)
    store = SimpleNamespace(layout=SimpleNamespace(num_kv_heads=2, head_size=256), pages=torch.zeros(1))
    q = torch.zeros(40, 2 * gqa, 256)
    prefill, req = [(0, 40, 40, 0)], [0]
    with pytest.raises(ValueError, match="at most"):
        pf.prefill_attention_fused(store, q, q, prefill, req, torch.zeros(1, 1), 0.1,
                                   pf.build_tiles(prefill, req, gqa, "cpu"))
    ok = pf.build_tiles(prefill, req, gqa, "cpu", tokens=pf.block_m(gqa, 256))
    with pytest.raises(RuntimeError, match="device tensors"):
        pf.prefill_attention_fused(store, q, q, prefill, req, torch.zeros(1, 1), 0.1, ok)
    with pytest.raises(ValueError, match="own-group"):
        pf.prefill_attention(store, q, q, prefill, req, torch.zeros(1, 1), 0.1, own_group_key=q)
