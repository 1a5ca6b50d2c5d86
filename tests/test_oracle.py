"""CPU: pin the oracle (the checker of every GPU parity test) before trusting it.

Each oracle function is checked against the outputs the reference's own code
wrote for the same seeded inputs (``tests/golden``, made by
``tests/golden/make_golden.py``) and against what the mathematics fixes on its
own (closed forms, invariants, brute force on tiny inputs), chosen so that a
dropped term, a wrong index or a transposed operand fails at least one check.
The invariant cases follow ``tests/echokv_vllm/test_quant.py:16-48`` and
``test_canary_controller.py:20-60`` of the reference.
"""

import numpy as np
import pytest

import scripts as S
from host_sim import golden, replay
from oracle import attention as OA
from oracle import canary as OC
from oracle import quant as OQ

QG = np.load(S.__file__.replace("scripts.py", "quant.npz"), allow_pickle=False)
CG = np.load(S.__file__.replace("scripts.py", "canary.npz"), allow_pickle=False)


# ---- quant.py ---------------------------------------------------------------
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_and_pack_match_reference_bytes(bits):
    xs, _ = S.quant_inputs()
    for shift, x in xs.items():
        tag = f"s{int(shift)}_b{bits}"
        c, sc, mn = OQ.quantize(x, bits, 32)
        assert np.array_equal(c, QG[f"codes_{tag}"])
        assert np.array_equal(sc.view(np.uint16), QG[f"scale_{tag}"].view(np.uint16))
        assert np.array_equal(mn.view(np.uint16), QG[f"min_{tag}"].view(np.uint16))
        assert np.array_equal(OQ.pack(c, bits), QG[f"packed_{tag}"])
        assert np.array_equal(OQ.unpack(OQ.pack(c, bits), bits), c)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_channel_stats_and_fake_quant_match_reference(bits):
    _, k = S.quant_inputs()
    sc, mn = OQ.stats_along(k[:32], bits, 0)
    assert np.array_equal(sc.view(np.uint16), QG[f"stats_scale_b{bits}"].view(np.uint16))
    assert np.array_equal(mn.view(np.uint16), QG[f"stats_min_b{bits}"].view(np.uint16))
    assert np.array_equal(OQ.fake_quant_channels(k, bits, 32), QG[f"fqc_b{bits}"])


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_invariants(bits):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((64, 128), dtype=np.float32) * 3
    x[3, :32] = -0.75  # constant group (an fp16 value: stored exactly)
    c, sc, mn = OQ.quantize(x, bits, 32)
    assert c.max() <= (1 << bits) - 1
    y = OQ.dequantize(c, sc, mn, 32)
    step = np.repeat(sc.astype(np.float32), 32, axis=-1)
    # within half a step of the input, up to the fp16 rounding of the min
    slack = np.repeat(np.abs(mn.astype(np.float32) - x.reshape(64, 4, 32).min(-1)), 32, axis=-1)
    assert np.all(np.abs(y - x) <= 0.5 * step + slack + 1e-6)
    assert np.array_equal(y[3, :32], x[3, :32])
    # the scale floor is the smallest normal fp16
    assert np.all(sc.astype(np.float32) >= 2.0 ** -14)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_groups_of_any_size_are_consecutive_channel_runs(bits):
    """V groups that are not powers of two (the reference takes any divisor of the
    head size): group j of size g is channels [j*g, (j+1)*g), each quantized as a
    row of its own -- a transposed grouping (channels j, j + D/g, ...) fails this.
    Group 32 is pinned to the reference's bytes above."""
    rng = np.random.default_rng(13)
    x = rng.standard_normal((8, 96), dtype=np.float32) * 2
    x[:, 5] += 9.0  # an outlier channel that moves one group's stats only
    for g in (96, 24, 12, 6, 3, 1):
        c, sc, mn = OQ.quantize(x, bits, g)
        assert sc.shape == (8, 96 // g)
        for j in range(96 // g):
            cj, scj, mnj = OQ.quantize(x[:, j * g : (j + 1) * g], bits, g)
            assert np.array_equal(c[:, j * g : (j + 1) * g], cj)
            assert np.array_equal(sc[:, j : j + 1].view(np.uint16), scj.view(np.uint16))
            assert np.array_equal(mn[:, j : j + 1].view(np.uint16), mnj.view(np.uint16))
        y = OQ.dequantize(c, sc, mn, g)
        assert np.all(np.abs(y - x) <= 0.5 * np.repeat(sc.astype(np.float32), g, axis=-1)
                      + np.repeat(np.abs(mn.astype(np.float32) - x.reshape(8, -1, g).min(-1)), g, axis=-1) + 1e-6)


def test_fake_quant_channels_keeps_partial_tail_exact():
    rng = np.random.default_rng(12)
    k = rng.standard_normal((40, 2, 16), dtype=np.float32)
    y = OQ.fake_quant_channels(k, 4, 16)
    assert np.array_equal(y[32:], k[32:])
    # whole groups equal the two-step round trip under their own channel stats
    sc, mn = OQ.stats_along(k[16:32], 4, 0)
    ref = OQ.dequantize_with(OQ.quantize_with(k[16:32], sc, mn, 4), sc, mn)
    assert np.array_equal(y[16:32], ref)


# ---- attention (decode.py:95-129, prefill.py:210-236) ------------------------
def test_attend_closed_forms():
    rng = np.random.default_rng(13)
    q = rng.standard_normal((4, 8))
    k = rng.standard_normal((1, 2, 8))
    v = rng.standard_normal((1, 2, 8))
    # one key: the output is its value, repeated over the GQA heads
    assert np.allclose(OA.attend(q, k, v, 0.3), np.repeat(v[0], 2, axis=0))
    # equal scores: the mean of the values
    k0 = np.zeros((5, 2, 8))
    v5 = rng.standard_normal((5, 2, 8))
    assert np.allclose(OA.attend(q, k0, v5, 1.0), np.repeat(v5.mean(0), 2, axis=0))
    # brute force per head (GQA: query head j reads KV head j // 2)
    k5 = rng.standard_normal((5, 2, 8))
    got = OA.attend(q, k5, v5, 0.5, limit=4)
    for j in range(4):
        s = np.array([0.5 * q[j] @ k5[t, j // 2] for t in range(4)])
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(got[j], sum(p[t] * v5[t, j // 2] for t in range(4)))


@pytest.fixture(scope="module")
def cfg1_sims():
    return {}


def _cfg1(cfg1_sims, name):
    if name not in cfg1_sims:
        cfg1_sims[name] = replay(next(s for s in S.all_scripts() if s.name == name))
    return cfg1_sims[name]


@pytest.mark.parametrize("name", ["cfg1_int8_bs16", "cfg1_int4_bs16", "cfg1_int2_bs16", "cfg1_int4_bs32"])
def test_decode_oracle_matches_reference_output(cfg1_sims, name):
    sim = _cfg1(cfg1_sims, name)
    s = sim.s
    q = S.cfg1_query(s).astype(np.float32)
    out = OA.decode_attention(sim.ps, q, s.meta["table"], s.meta["lens"], s.d ** -0.5, vectorized=True)
    ref = golden(name)["decode_out"]
    assert np.abs(out - ref).max() < 2e-5


def test_prefill_oracle_and_gather_match_reference_output(cfg1_sims):
    sim = _cfg1(cfg1_sims, "cfg1_int4_bs16")
    s, g = sim.s, golden("cfg1_int4_bs16")
    pos = np.arange(64)
    k, v = sim.ps.gather(np.asarray(s.meta["table"][0], np.int64)[pos // s.bs], pos % s.bs)
    assert np.array_equal(k, g["gather0_k"]) and np.array_equal(v, g["gather0_v"])
    prefill, req_of, pq = S.cfg1_prefill(s)
    out = OA.prefill_attention(sim.ps, pq, prefill, req_of, s.meta["table"], s.d ** -0.5)
    assert np.abs(out - g["prefill_out"]).max() < 2e-5
    vec = OA.prefill_attention(sim.ps, pq, prefill, req_of, s.meta["table"], s.d ** -0.5, vectorized=True)
    assert np.abs(vec - g["prefill_out"]).max() < 2e-5
    assert np.abs(vec - out).max() < 1e-12  # the blocked form computes the loop's values


def test_blocked_causal_attention_equals_per_query_loop():
    """attend_causal (one matrix product per head) against attend with the
    bottom-right limit, query by query, on GQA 3 and a chunk shorter than the context."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((7, 6, 16))
    k = rng.standard_normal((20, 2, 16))
    v = rng.standard_normal((20, 2, 16))
    got = OA.attend_causal(q, k, v, 0.3)
    for i in range(7):
        ref = OA.attend(q[i], k, v, 0.3, limit=20 - 7 + i + 1)
        assert np.abs(got[i] - ref).max() < 1e-12
    # the last query sees every key; the first sees 14
    assert np.abs(got[6] - OA.attend(q[6], k, v, 0.3)).max() < 1e-12


# ---- canary.py:59-89 -----------------------------------------------------------
def test_canary_oracle_matches_reference_outputs():
    (q, kref), (q2, kref2) = S.canary_inputs()
    assert np.allclose(OC.canary_kl(q, kref, (2, 4, 8), 32, 64 ** -0.5), CG["small_out"], rtol=1e-4, atol=1e-7)
    assert np.allclose(OC.canary_kl(q2, kref2, (2, 4, 8), 16, 128 ** -0.5), CG["cfg_out"], rtol=1e-4, atol=1e-7)


def test_canary_closed_forms():
    rng = np.random.default_rng(14)
    q = rng.standard_normal((3, 4, 16)).astype(np.float32)
    # keys every tier stores exactly (levels 0 and 255 = 3*5*17: the scale 255/L is
    # an integer for L = 3, 15, 255) give KL = 0
    k = np.where(rng.random((32, 2, 16)) < 0.5, 0.0, 255.0).astype(np.float32)
    assert np.all(OC.canary_kl(q, k, (2, 4, 8), 16, 0.01) == 0)
    # otherwise KL >= 0 and shrinks with more bits
    k = rng.standard_normal((64, 2, 16)).astype(np.float32) * 4
    d = OC.canary_kl(q, k, (2, 4, 8), 16, 0.25)
    assert d[0] > d[1] > d[2] >= 0
    # only the newest whole groups count: older keys do not change the result
    k2 = np.concatenate([rng.standard_normal((7, 2, 16)).astype(np.float32), k])
    assert np.array_equal(OC.canary_kl(q, k2, (2, 4, 8), 16, 0.25), d)
    with pytest.raises(ValueError):
        OC.canary_kl(q, k[:15], (4,), 16, 0.25)
