"""CPU: the native per-step driver (``ekh_stepper_run`` behind ``StepDriver``).

The driver folds the builder's whole host step into one native call: the batch
layout, the write plan, the blocks that open in every layer's pool at that
layer's tier, the seal rows of evicted groups and the image the device reads.
Each part is pinned against what it replaces:

* the plan, opened blocks, page headers, demotion victims and seal rows equal
  the per-layer composition of the planner and pools (``WritePlanner.plan``,
  ``ChunkPool.fresh_opens`` / ``open`` / ``seal_row``, ``SharedState.commit``),
  whose decisions the reference's golden page bytes pin (tests/test_store_host.py),
  step by step on random serving streams under pool pressure and slot eviction;
* the batch layout follows the reference builder's rules
  (``echokv_vllm/backend.py:372-392``), restated below over numpy;
* the image keeps its graph-visible parts at fixed offsets.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from echokv_amd import _host
from echokv_amd.step import StepDriver
from echokv_amd.tiered_cache import ChunkPool, TieredLayout
from echokv_amd.write_plan import SharedState


def batches(rng, bs, n_blocks, steps, max_live, decode_only_every=3):
    """Serving-like steps: (query starts, lengths, slots) per step. Requests arrive
    with a chunked prefill, decode one token per step, finish and free their blocks;
    every few steps is decode-only with graph padding (length 0, slot -1)."""
    free = list(rng.permutation(n_blocks))
    live = []  # [blocks, length]
    for step in range(steps):
        while len(live) < max_live and len(free) > 4 and rng.random() < 0.5:
            live.append([[], 0])
        decode_only = step % decode_only_every == 0
        qlens, lens, slots = [], [], []
        for sq in list(live):
            if sq[1] and rng.random() < 0.05:  # finishes
                free.extend(sq[0])
                live.remove(sq)
                continue
            n = 1 if decode_only or sq[1] else int(rng.integers(2, 3 * bs))
            if rng.random() < 0.15:
                n = 0  # not scheduled this step
            toks = []
            for _ in range(n):
                if sq[1] % bs == 0:
                    if not free:
                        break
                    sq[0].append(free.pop(0))
                toks.append(sq[0][sq[1] // bs] * bs + sq[1] % bs)
                sq[1] += 1
            qlens.append(len(toks))
            lens.append(sq[1])
            slots += toks
        if decode_only:  # graph padding requests
            pad = int(rng.integers(0, 3))
            qlens += [1] * pad
            lens += [0] * pad
            slots += [-1] * pad
        qsl = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
        yield qsl, np.array(lens, np.int32), np.array(slots, np.int64)


def reference_layout(qsl, lens, t, nq, fire):
    """The reference builder's batch layout (backend.py:372-392), over numpy."""
    qlen = np.diff(qsl.astype(np.int64))
    lens = lens.astype(np.int64)
    live = (qlen > 0) & (lens > 0)
    d_idx = np.arange(lens.size) if (qlen <= 1).all() else np.flatnonzero(live & (qlen == 1))
    d_lens = np.where(qlen[d_idx] == 1, lens[d_idx], 0)
    d_rows = np.minimum(qsl[:-1][d_idx], max(t - 1, 0))
    prefill = [(int(qsl[r]), int(qsl[r + 1]), int(lens[r]), int(r)) for r in np.flatnonzero(live & (qlen > 1))]
    last = (qsl[1:] - 1)[live][:nq] if fire else np.zeros(0, np.int64)
    ctx = float(lens[live][: last.size].mean()) if last.size else 0.0
    return (d_rows, d_idx, d_lens), prefill, last, ctx


class Group:
    def __init__(self, layout, n_layers, n_blocks, slots, window):
        self.shared = SharedState(n_blocks, layout.block_size, layout.k_group, slots, window, "cpu")
        self.pools = [ChunkPool(layout, n_blocks, self.shared) for _ in range(n_layers)]


@pytest.mark.parametrize("bs,kg,mem,slots,seed", [(16, 16, 4, 6, 0), (32, 16, 8, 4, 1), (16, 16, 8, 3, 2),
                                                  (64, 32, 4, 5, 3)])
def test_stepper_equals_the_planner_and_pools_composed(bs, kg, mem, slots, seed):
    rng = np.random.default_rng(seed)
    n_layers, n_blocks, window, nq, cap = 3, 40, 2 * kg, 4, 24
    layout = TieredLayout(2, 64, bs, mem, kg, 32)
    old = Group(layout, n_layers, n_blocks, slots, window)
    new = Group(layout, n_layers, n_blocks, slots, window)
    driver = StepDriver(new.shared, [SimpleNamespace(pool=p) for p in new.pools], cap, nq, "cpu")
    seen = dict(steps=0, opens=0, victims=0, seals=0, prefill=0, oversized=0)
    for step, (qsl, lens, sm) in enumerate(batches(rng, bs, n_blocks, 120, max_live=slots)):
        tiers = rng.choice([2, 4, 8], n_layers).astype(np.int32)
        fire = step % 5 == 0
        msg = f"seed {seed} step {step}"
        # The composition the stepper replaces.
        try:
            plan = old.shared.planner.plan(sm)
        except RuntimeError:
            with pytest.raises(RuntimeError):
                driver.run(qsl, lens, sm, tiers, fire)
            break
        opens = old.pools[0].fresh_opens(plan)
        seals, headers, victims = [], [], []
        for li, pool in enumerate(old.pools):
            seals.append([pool.seal_row(e) for e in plan.evictions if e.fill > 0])
            if opens.size:
                got = []
                _, h = pool.open(opens, int(tiers[li]), plan.touched_np, got.extend)
                headers.append(h)
                victims += [(li, b) for b in got]
        old.shared.commit(plan)

        up = driver.run(qsl, lens, sm, tiers, fire)
        t = sm.size
        np.testing.assert_array_equal(up.tok.numpy(), np.stack([plan.tok_slot, plan.tok_res, plan.tok_sealed,
                                                                plan.tok_kref]), err_msg=msg)
        assert up.n_fin == plan.n_fin and int(up.fin_count) == plan.n_fin, msg
        np.testing.assert_array_equal(up.fin[: plan.n_fin].numpy(), plan.fin, err_msg=msg)
        blocks, values, gslots, groups = (x.numpy() for x in up.res_map)
        np.testing.assert_array_equal(blocks, plan.res_map_block, err_msg=msg)
        np.testing.assert_array_equal(values, plan.res_map_value, err_msg=msg)
        np.testing.assert_array_equal(gslots, plan.res_group_slot, err_msg=msg)
        np.testing.assert_array_equal(groups, plan.res_group_value, err_msg=msg)
        np.testing.assert_array_equal(up.open_ids.numpy(), opens, err_msg=msg)
        if opens.size:
            want = np.concatenate([np.ascontiguousarray(h).view(np.int64).reshape(-1) for h in headers])
            np.testing.assert_array_equal(up.headers.numpy(), want, err_msg=msg)
        assert [(int(a), int(b)) for a, b in up.victims] == victims, msg
        for li in range(n_layers):
            got = up.seal_rows[li].numpy().tolist() if up.seal_rows else []
            assert got == seals[li], msg
        for li in range(n_layers):
            assert np.array_equal(old.pools[li].tag_h, new.pools[li].tag_h), msg
            assert old.pools[li].free == new.pools[li].free, msg
            assert old.pools[li].live_tiers() == new.pools[li].live_tiers(), msg
            live = old.pools[li].live_tiers()  # the tiers the layer's decode runs passes for
            assert int(up.tier_masks[li, 0]) == sum(b for b in (2, 4, 8) if live[b]), msg
            assert int(up.host_tier_masks[li]) == int(up.tier_masks[li, 0]), msg
        assert np.array_equal(old.shared.cum_h, new.shared.cum_h) and np.array_equal(old.shared.last_h,
                                                                                      new.shared.last_h), msg

        (d_rows, d_idx, d_lens), prefill, last, ctx = reference_layout(qsl, lens, t, nq, fire)
        if d_idx.size:
            got = [x.numpy() for x in up.decode]
            np.testing.assert_array_equal(got[0], d_rows, err_msg=msg)
            np.testing.assert_array_equal(got[1], d_idx, err_msg=msg)
            np.testing.assert_array_equal(got[2], d_lens, err_msg=msg)
        else:
            assert up.decode is None, msg
        assert up.prefill == prefill, msg
        assert up.n_canary == last.size and up.canary_rows[: last.size].tolist() == last.tolist(), msg
        assert up.canary_ctx == pytest.approx(ctx), msg

        seen["steps"] += 1
        seen["opens"] += int(opens.size)
        seen["victims"] += len(victims)
        seen["seals"] += sum(map(len, seals))
        seen["prefill"] += len(prefill)
        seen["oversized"] += max(d_idx.size, t, plan.n_fin) > driver.cap
    print(f"[stepper] {seen}")
    assert seen["steps"] >= 60 and seen["opens"] and seen["prefill"]
    if mem == 4:
        assert seen["victims"], "pool pressure must demote blocks"


def test_graph_visible_parts_keep_their_addresses():
    layout = TieredLayout(2, 64, 16, 8, 16, 32)
    g = Group(layout, 2, 32, 4, 16)
    driver = StepDriver(g.shared, [SimpleNamespace(pool=p) for p in g.pools], cap=8, canary_slots=3, device="cpu")
    tiers = np.array([4, 8], np.int32)
    # A 2-request decode step, then a 3-request one: same addresses.
    a = driver.run(np.array([0, 1, 2], np.int32), np.array([1, 1], np.int32), np.array([0, 16], np.int64), tiers,
                   False)
    b = driver.run(np.array([0, 1, 2, 3], np.int32), np.array([2, 2, 1], np.int32), np.array([1, 17, 32], np.int64),
                   tiers, True)
    for x, y in ((a.tok, b.tok), (a.fin, b.fin), (a.fin_count, b.fin_count), (a.canary_rows, b.canary_rows),
                 (a.tier_masks, b.tier_masks)):
        assert x.data_ptr() == y.data_ptr()
    assert a.tier_masks[:, 0].tolist() == [4, 8]  # each layer opened its blocks at its own tier
    assert a.decode[0].data_ptr() == b.decode[0].data_ptr() and a.decode[2].data_ptr() == b.decode[2].data_ptr()
    assert a.tok.stride(0) == b.tok.stride(0) == 8  # token rows stride by the capacity
    assert b.decode[2].tolist() == [2, 2, 1] and b.canary_rows.tolist() == [0, 1, 2] and b.n_canary == 3
    # A step past the capacity (a 20-token prefill) gets a buffer of its own.
    c = driver.run(np.array([0, 20], np.int32), np.array([20], np.int32), np.arange(48, 68, dtype=np.int64), tiers,
                   False)
    assert c.tok.data_ptr() != a.tok.data_ptr() and c.tok.shape == (4, 20) and c.prefill == [(0, 20, 20, 0)]
    assert c.tok[0].tolist() == list(range(48, 68))


def test_stepper_refuses_bad_batches():
    layout = TieredLayout(2, 64, 16, 8, 16, 32)
    g = Group(layout, 1, 8, 4, 16)
    driver = StepDriver(g.shared, [SimpleNamespace(pool=g.pools[0])], cap=8, canary_slots=2, device="cpu")
    ok = np.array([4], np.int32)
    with pytest.raises(ValueError):  # a slot past the pool
        driver.run(np.array([0, 1], np.int32), np.array([1], np.int32), np.array([16 * 8], np.int64), ok, False)
    with pytest.raises(ValueError):  # query starts past the tokens
        driver.run(np.array([0, 3], np.int32), np.array([3], np.int32), np.array([0], np.int64), ok, False)
    with pytest.raises(ValueError):  # an unsupported tier
        driver.run(np.array([0, 1], np.int32), np.array([1], np.int32), np.array([0], np.int64),
                   np.array([3], np.int32), False)
    other = SharedState(8, 16, 16, 4, 16, "cpu")
    with pytest.raises(ValueError):  # a pool of another planner
        StepDriver(other, [SimpleNamespace(pool=g.pools[0])], 8, 2, "cpu")


def test_host_slots_native_matches_the_formula():
    rng = np.random.default_rng(7)
    table = rng.integers(0, 1000, (6, 9)).astype(np.int32)
    qsl = np.array([0, 1, 5, 5, 12], np.int32)
    lens = np.array([30, 40, 7, 100], np.int32)
    t = 14
    slots = np.empty(t, np.int64)
    row_map = np.array([5, 0, 3, 2], np.int64)
    batch = _host.Batch(4, t, qsl.ctypes.data, lens.ctypes.data, None)
    import ctypes as C
    rc = _host.lib().ekh_host_slots(C.byref(batch), table.ctypes.data, 6, 9, 9, row_map.ctypes.data, 4, 16,
                                    slots.ctypes.data)
    assert rc == _host.OK
    want = []
    for r in range(4):
        for i in range(qsl[r], qsl[r + 1]):
            pos = lens[r] - (qsl[r + 1] - qsl[r]) + (i - qsl[r])
            want.append(int(table[row_map[r], pos // 16]) * 16 + pos % 16)
    assert slots.tolist() == want + [-1, -1]
    lens[3] = 200  # position 199 -> block 12, past the table's 9 columns
    assert _host.lib().ekh_host_slots(C.byref(batch), table.ctypes.data, 6, 9, 9, row_map.ctypes.data, 4, 16,
                                      slots.ctypes.data) == _host.EINVAL
