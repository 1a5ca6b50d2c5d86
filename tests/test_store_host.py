"""CPU: host planner + chunk pool (product) driving the oracle's device effects
reproduce the reference store's page bytes, residual state, K_ref ring, write
plans and counters after every golden script.

Mirrors ``tests/echokv_vllm/test_tiered_cache.py`` and ``test_step_path.py``
of the reference, against the bytes its own store wrote (``tests/golden``)."""

import hashlib

import numpy as np
import pytest

import scripts as S
from host_sim import golden, replay

SMALL = [s.name for s in S.small_scripts()]
CFG1 = [s.name for s in S.all_scripts() if s.name.startswith("cfg1")]


def _script(name):
    return next(s for s in S.all_scripts() if s.name == name)


@pytest.fixture(scope="module")
def sims():
    return {}


def _sim(sims, name):
    if name not in sims:
        sims[name] = replay(_script(name))
    return sims[name]


@pytest.mark.parametrize("name", SMALL)
def test_pages_match_reference_bytes(sims, name):
    sim, g = _sim(sims, name), golden(name)
    got = sim.ps.pages
    exp = g["pages"]
    bad = np.flatnonzero((got != exp).any(axis=1))
    assert bad.size == 0, f"pages {bad.tolist()} differ"
    assert bool(g["guard_ok"])


@pytest.mark.parametrize("name", SMALL + CFG1)
def test_residual_map_and_rows(sims, name):
    sim, g = _sim(sims, name), golden(name)
    np.testing.assert_array_equal(sim.ps.block_res, g["block_res"])
    np.testing.assert_array_equal(sim.ps.res_group, g["res_group"])
    live = sim.ps.block_res[sim.ps.block_res >= 0]
    np.testing.assert_array_equal(live, g["res_live_slots"])
    np.testing.assert_array_equal(sim.ps.res_k[live], g["res_live"])


@pytest.mark.parametrize("name", SMALL + CFG1)
def test_counters_and_tags(sims, name):
    sim, g = _sim(sims, name), golden(name)
    np.testing.assert_array_equal(sim.counters(), g["counters"])
    np.testing.assert_array_equal(sim.ps.pages[:, 0], g["tags"])


@pytest.mark.parametrize("name", SMALL)
def test_write_plans_match(sims, name):
    sim, g = _sim(sims, name), golden(name)
    for i, (plan, opened) in enumerate(sim.plans):
        tok = np.stack([plan.tok_slot, plan.tok_res, plan.tok_sealed, plan.tok_kref])
        np.testing.assert_array_equal(tok, g[f"plan{i}_tok"], err_msg=f"step {i}")
        np.testing.assert_array_equal(plan.fin, g[f"plan{i}_fin"], err_msg=f"step {i}")
        ev = np.array([[e.slot, e.block, e.group, e.fill] for e in plan.evictions], np.int64).reshape(-1, 4)
        np.testing.assert_array_equal(ev, g[f"plan{i}_evict"], err_msg=f"step {i}")
        hdr = np.zeros((0, 17), np.int64) if opened is None else np.concatenate(
            [opened[0][:, None], opened[1].astype(np.int64)], 1)
        np.testing.assert_array_equal(hdr, g[f"plan{i}_open"], err_msg=f"step {i}")


@pytest.mark.parametrize("name", CFG1)
def test_cfg1_page_hashes(sims, name):
    sim, g = _sim(sims, name), golden(name)
    got = np.array([hashlib.sha256(sim.ps.pages[b].tobytes()).hexdigest() for b in range(sim.ps.n)])
    bad = np.flatnonzero(got != g["page_sha"])
    assert bad.size == 0, f"pages {bad.tolist()} differ"


def test_step_path_kref_ring(sims):
    sim, g = _sim(sims, "step_path"), golden("step_path")
    np.testing.assert_array_equal(sim.kref, g["kref"])
    assert sim.planner.kref_pos == int(g["kref_pos"]) and sim.planner.kref_fill == int(g["kref_fill"])


def test_known_answers_of_the_reference_store_tests(sims):
    """The behaviours the reference asserts (test_tiered_cache.py:100-230)."""
    assert [int(t) for t in _sim(sims, "pool_exhaustion").ps.pages[:, 0]] == [8] * 4 + [2] * 8
    pe = _sim(sims, "pool_exhaustion")
    assert pe.pool.downgraded_blocks == 8 and len(pe.pool.free) == 0
    ld = _sim(sims, "lru_demote")
    assert int(ld.ps.pages[1, 0]) == 8 and int(ld.ps.pages[0, 0]) == 2 and ld.pool.demoted_blocks == 1
    assert len(ld.pool.free) == 1
    nv = _sim(sims, "no_victim_lower")
    assert [int(nv.ps.pages[b, 0]) for b in (0, 1)] == [8, 4] and nv.pool.demoted_blocks == 0
    ro = _sim(sims, "reopen")
    assert len(ro.planner.free) == 16
    ev = _sim(sims, "eviction_seal")
    assert ev.pool.sealed_groups == 1 and int(ev.ps.pages[0, 1]) == 1
    assert len(_sim(sims, "decode_one_token").planner.free) == 15
    assert len(_sim(sims, "uniform_int4").planner.free) == 16


def test_triton_interpreter_bytes_agree():
    """The reference's Triton write kernels under the CPU interpreter wrote the same pages
    as its PyTorch path for every script (hashes recorded by make_golden.py)."""
    import json

    p = S.__file__.replace("scripts.py", "triton_interp_hashes.json")
    try:
        tri = json.load(open(p))
    except FileNotFoundError:
        pytest.skip("no Triton-interpreter hashes recorded")
    man = json.load(open(p.replace("triton_interp_hashes.json", "manifest.json")))
    assert tri, "empty Triton hash record"
    for name, h in tri.items():
        assert h["triton_pages_sha"] == man[name]["pages_sha"], name


@pytest.mark.parametrize("name", ["tier_change", "eviction_seal", "cfg1_int4_bs16", "pool_exhaustion"])
def test_vectorized_gather_equals_loop(sims, name):
    sim = _sim(sims, name)
    rng = np.random.default_rng(0)
    blk = rng.integers(0, sim.ps.n, 300)
    off = rng.integers(0, sim.s.bs, 300)
    k1, v1 = sim.ps.gather(blk, off)
    k2, v2 = sim.ps.gather_vec(blk, off)
    np.testing.assert_array_equal(k1, k2)
    np.testing.assert_array_equal(v1, v2)
