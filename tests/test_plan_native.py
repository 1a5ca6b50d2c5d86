"""CPU: the native write planner (libechokv_host.so) against the plain-Python
planner of the oracle, which is itself pinned to the reference's own plans.

1. ``oracle.plan.PlannerOracle`` reproduces every golden script's per-step token
   table, fin rows and evictions (written by the reference's ``WritePlanner``).
2. On random step streams -- decode steps, chunked prefills, sequences finishing
   and their blocks reused (reopened at offset 0), few residual slots so slots are
   evicted and groups sealed, several K groups per block -- the native planner's
   plans, residual-map updates, free list and K_ref cursor equal the oracle's, step
   by step. (The reference's planner is exercised the same way by
   tests/echokv_vllm/test_step_path.py:35-71.)
"""

import numpy as np
import pytest

import scripts as S
from echokv_amd.write_plan import SharedState, WritePlanner
from host_sim import golden
from oracle.plan import PlannerOracle


@pytest.mark.parametrize("name", [s.name for s in S.small_scripts()])
def test_oracle_planner_reproduces_reference_plans(name):
    s = next(x for x in S.all_scripts() if x.name == name)
    g = golden(name)
    po = PlannerOracle(s.bs, s.kg, s.residual_slots, s.kg)
    for i, (slots, _, _, _) in enumerate(S.script_inputs(s)):
        tok, fin, ev, _, _ = po.plan(slots)
        np.testing.assert_array_equal(tok, g[f"plan{i}_tok"], err_msg=f"step {i}")
        np.testing.assert_array_equal(fin, g[f"plan{i}_fin"], err_msg=f"step {i}")
        np.testing.assert_array_equal(ev, g[f"plan{i}_evict"], err_msg=f"step {i}")


def random_stream(rng, bs, n_blocks, n_seqs, steps, writers):
    """Slot mappings of a serving-like run over ``n_blocks`` pages: ``n_seqs`` live
    sequences, at most ``writers`` of them writing in a step (each leaves at most
    one K group open), so idle sequences hold residual slots that later steps evict."""
    free_blocks = list(rng.permutation(n_blocks))
    seqs = []  # [blocks, length]
    out = []
    for _ in range(steps):
        while len(seqs) < n_seqs and free_blocks:
            seqs.append([[], 0])
        rows = []
        pick = rng.permutation(len(seqs))[: int(rng.integers(1, writers + 1))]
        for i in sorted(pick.tolist(), reverse=True):
            sq = seqs[i]
            r = rng.random()
            if r < 0.1 and sq[1] > 0:  # finishes: its blocks return to the free list
                free_blocks.extend(sq[0])
                seqs.pop(i)
                continue
            n = int(rng.integers(1, 3 * bs)) if r < 0.3 else 1  # a prefill chunk or a decode token
            for _ in range(n):
                if sq[1] % bs == 0:
                    if not free_blocks:
                        break
                    sq[0].append(free_blocks.pop(0))
                rows.append(sq[0][sq[1] // bs] * bs + sq[1] % bs)
                sq[1] += 1
        rows += [-1] * int(rng.integers(0, 3))  # padding rows, as CUDA-graph batches carry
        rng.shuffle(rows)
        out.append(np.array(rows, np.int64))
    return out


@pytest.mark.parametrize("bs,kg,slots,seed", [(16, 16, 3, 0), (16, 8, 4, 1), (32, 8, 6, 2), (32, 16, 2, 3),
                                             (64, 16, 5, 4), (16, 4, 2, 5)])
def test_native_planner_equals_oracle_on_random_streams(bs, kg, slots, seed):
    rng = np.random.default_rng(seed)
    n_blocks, window = 48, 2 * kg
    native = WritePlanner(bs, kg, slots, window, num_blocks=n_blocks)
    po = PlannerOracle(bs, kg, slots, window)
    evicted = sealed = steps = 0
    # Groups get slots in block order, so a slot a later group of the same step
    # frees cannot serve an earlier one: keep the writers well under the slots.
    for step, sm in enumerate(random_stream(rng, bs, n_blocks, 3 * slots, 80, max(1, slots // 2))):
        try:
            tok, fin, ev, opened, res_log = po.plan(sm)
        except RuntimeError:
            with pytest.raises(RuntimeError):
                native.plan(sm)
            break
        plan = native.plan(sm)
        steps += 1
        msg = f"seed {seed} step {step}"
        np.testing.assert_array_equal(np.stack([plan.tok_slot, plan.tok_res, plan.tok_sealed, plan.tok_kref]), tok,
                                      err_msg=msg)
        np.testing.assert_array_equal(plan.fin, fin, err_msg=msg)
        got_ev = np.array([[e.slot, e.block, e.group, e.fill] for e in plan.evictions], np.int64).reshape(-1, 4)
        np.testing.assert_array_equal(got_ev, ev, err_msg=msg)
        np.testing.assert_array_equal(plan.open_np, opened, err_msg=msg)
        res = dict(res_log)  # first appearance order, last value wins
        assert plan.res_map_block.tolist() == list(res), msg
        assert plan.res_map_value.tolist() == list(res.values()), msg
        assert native.free == po.stack, msg
        assert (native.kref_pos, native.kref_fill) == (po.kref_pos, po.kref_fill), msg
        evicted += len(ev)
        sealed += int(tok[2].sum())
    print(f"[planner] bs {bs} kg {kg} slots {slots}: {steps} steps, {evicted} evictions, {sealed} sealed-group writes")
    assert steps >= 60 and evicted > 0 and sealed > 0, "the stream must exercise evictions and sealed groups"


def test_both_planners_refuse_more_open_groups_than_slots():
    sm = np.array([16 * b + 3 for b in range(5)])  # five partial groups, four slots
    with pytest.raises(RuntimeError):
        PlannerOracle(16, 16, 4, 16).plan(sm)
    with pytest.raises(RuntimeError, match="open K groups"):
        WritePlanner(16, 16, 4, 16, num_blocks=8).plan(sm)


def test_shared_state_commit_and_views():
    sh = SharedState(8, 16, 16, 4, kref_window=16, device="cpu")
    plan = sh.planner.plan(np.array([16 * 3 + 0, 16 * 3 + 1, 16 * 5 + 7, -1]))
    sh.commit(plan)
    assert sh.fill_h.tolist() == [0, 0, 0, 2, 0, 8, 0, 0]
    assert sh.cum_h.tolist() == [0, 0, 0, 2, 0, 1, 0, 0]
    assert sh.last_h[3] == plan.step == 1
    fill = sh.fill_h  # a view of native memory that outlives the SharedState object
    del sh, plan
    assert fill.tolist() == [0, 0, 0, 2, 0, 8, 0, 0]
    with pytest.raises(ValueError):
        SharedState(8, 16, 16, 4, kref_window=16, device="cpu").planner.plan(np.array([16 * 8]))
