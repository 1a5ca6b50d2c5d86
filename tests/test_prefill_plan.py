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
