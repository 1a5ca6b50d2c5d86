"""Seeded write scripts shared by the golden-fixture generator and the tests.

A script is a sequence of store writes (slot mapping + target tier per step)
on one layer's paged store. K/V values come from ``numpy.random.default_rng``
so every consumer (the generator here, the CPU oracle tests, the GPU parity
tests on a box without the reference) rebuilds identical inputs from the seed.

The scripts mirror the reference's own store tests
(``tests/echokv_vllm/test_tiered_cache.py:100-230``,
``tests/echokv_vllm/test_step_path.py:26-33``) plus the BASELINE config-1
shape (4 sequences, 32 query / 8 KV heads, head_dim 128, page block 16).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Script:
    name: str
    h: int
    d: int
    bs: int
    mem_bits: int
    kg: int
    vg: int
    num_blocks: int
    residual_slots: int
    steps: list  # [(slots int64 [n], target bits)]
    seed: int = 0
    dtype: str = "f32"  # K/V (and residual) dtype: f32 or f16
    kref_window: int | None = None  # None: no K_ref ring written
    outliers: tuple = ((1, 30.0),)  # (channel, offset) added to K
    row_pad: int = 0
    full_bytes: bool = True  # fixture keeps whole pages (else per-page hashes)
    meta: dict = field(default_factory=dict)


def kv_for_step(rng: np.random.Generator, s: Script, n: int):
    """K and V ``[n, H, D]`` for one step, in the script's dtype."""
    k = rng.standard_normal((n, s.h, s.d), dtype=np.float32)
    for ch, off in s.outliers:
        k[..., ch] += np.float32(off)
    v = rng.standard_normal((n, s.h, s.d), dtype=np.float32)
    if s.dtype == "f16":
        return k.astype(np.float16), v.astype(np.float16)
    return k, v


def iter_inputs(s: Script):
    """(slots, bits, k, v) for each step of ``s``."""
    rng = np.random.default_rng(s.seed)
    for slots, bits in s.steps:
        k, v = kv_for_step(rng, s, slots.size)
        yield slots, bits, k, v


def _ar(a, b):
    return np.arange(a, b, dtype=np.int64)


def small_scripts() -> list[Script]:
    H, D, BS, KG, VG = 2, 64, 64, 32, 32
    out = []

    def mk(name, mem, nb, steps, **kw):
        out.append(Script(name, H, D, BS, mem, KG, VG, nb, kw.pop("residual_slots", 16), steps, **kw))

    for bits in (2, 4, 8):
        mk(f"uniform_int{bits}", 8, 6, [(_ar(0, 6 * BS), bits)], seed=bits)
    mk("tier_change", 8, 6, [(_ar(b * BS, (b + 1) * BS), t) for b, t in enumerate([8, 2, 4, 8, 2, 4])], seed=11)
    mk("decode_one_token", 8, 3, [(np.array([t], np.int64), [4, 8, 2][t % 3]) for t in range(2 * BS + 40)], seed=12)
    mk("prefill_then_decode", 8, 2, [(_ar(0, 20), 4), (_ar(20, 50), 4), (_ar(50, BS), 4)], seed=13)
    mk("pool_exhaustion", 4, 12, [(_ar(0, 12 * BS), 8)], seed=14, row_pad=48)
    mk("lru_demote", 4, 4, [(_ar(0, BS), 8), (_ar(BS, 2 * BS), 8)], seed=15)
    mk("no_victim_lower", 4, 4, [(_ar(0, 40), 8), (_ar(BS, 2 * BS), 8)], seed=16)
    mk("reopen", 8, 4, [(_ar(0, 3 * BS + 10), 8), (_ar(3 * BS, 4 * BS), 2), (_ar(0, BS), 2)], seed=17)
    a = _ar(3 * BS, 3 * BS + 21)
    b = _ar(7 * BS, 7 * BS + 37)
    order = np.random.default_rng(0).permutation(a.size + b.size)
    mk("interleaved", 6, 10, [(np.concatenate([a, b])[order], 4)], seed=18)
    mk("eviction_seal", 8, 6,
       [(_ar(bb * BS, bb * BS + 5), 8) for bb in range(3)] + [(_ar(5, BS), 8)], seed=19, residual_slots=2)
    # The per-step decode path: a prefill of two requests, then 60 decode steps
    # that complete groups from the residual and cross into new blocks; tiers
    # change every 7 steps; the K_ref ring (one K group wide) records every key.
    steps = [(np.r_[np.arange(40), 3 * BS + np.arange(10)].astype(np.int64), 8)]
    for i in range(60):
        aa, bb = 40 + i, 10 + i
        steps.append((np.array([[0, 5][aa // BS] * BS + aa % BS, [3, 6][bb // BS] * BS + bb % BS], np.int64),
                      (8, 4, 2)[((i + 1) // 7) % 3]))
    mk("step_path", 8, 8, steps, seed=20, residual_slots=8, kref_window=KG)
    return out


CFG1_LENS = (256, 512, 1000, 1024)
CFG1_OUTLIERS = tuple((c, 0.0) for c in (5, 37, 69, 101))  # scaled x8, see cfg1_kv


def cfg1_script(bits: int, bs: int = 16, kg: int = 16, seed: int = 0) -> Script:
    """4 sequences, H=8, D=128, fp16, prefill then one decode step.

    Pages are a seeded permutation (block table); the prefill writes ctx-1
    tokens of every sequence in one step, the decode step writes the last
    token of each. K channels 5, 37, 69, 101 are scaled x8 (outliers).
    """
    h, d = 8, 128
    lens = CFG1_LENS
    nbs = [-(-n // bs) for n in lens]
    num_blocks = sum(nbs) + 5
    perm = np.random.default_rng(seed + 1000).permutation(num_blocks)
    table = np.zeros((len(lens), max(nbs)), np.int64)
    o = 0
    for i, nb in enumerate(nbs):
        table[i, :nb] = perm[o : o + nb]
        o += nb
    pre = np.concatenate([table[i][np.arange(n - 1) // bs] * bs + np.arange(n - 1) % bs for i, n in enumerate(lens)])
    dec = np.array([table[i][(n - 1) // bs] * bs + (n - 1) % bs for i, n in enumerate(lens)], np.int64)
    s = Script(f"cfg1_int{bits}_bs{bs}", h, d, bs, 8, kg, 32, num_blocks, 8, [(pre.astype(np.int64), bits), (dec, bits)],
               seed=seed, dtype="f16", outliers=(), full_bytes=False)
    s.meta = {"table": table, "lens": np.array(lens, np.int64)}
    return s


def cfg1_kv(rng: np.random.Generator, s: Script, n: int):
    k = rng.standard_normal((n, s.h, s.d), dtype=np.float32)
    k[..., [5, 37, 69, 101]] *= np.float32(8.0)
    v = rng.standard_normal((n, s.h, s.d), dtype=np.float32)
    return k.astype(np.float16), v.astype(np.float16)


def script_inputs(s: Script):
    """(slots, bits, k, v) per step for any script (cfg1 uses its outlier rule)."""
    if s.name.startswith("cfg1"):
        rng = np.random.default_rng(s.seed)
        for slots, bits in s.steps:
            k, v = cfg1_kv(rng, s, slots.size)
            yield slots, bits, k, v
    else:
        yield from iter_inputs(s)


def cfg1_query(s: Script, hq: int = 32) -> np.ndarray:
    return np.random.default_rng(s.seed + 7).standard_normal((len(CFG1_LENS), hq, s.d), dtype=np.float32).astype(np.float16)


def all_scripts() -> list[Script]:
    return small_scripts() + [cfg1_script(b) for b in (8, 4, 2)] + [cfg1_script(4, bs=32, kg=32)]


def quant_inputs():
    """Seeded inputs of the quantization fixture: {shift: x [16, 4, 128] f32}."""
    rng = np.random.default_rng(5)
    xs = {}
    for shift in (0.0, 40.0, -40.0):
        x = rng.standard_normal((16, 4, 128), dtype=np.float32) + np.float32(shift)
        x[0, 0, :32] = 1.25  # a constant group
        xs[shift] = x
    k = rng.standard_normal((70, 2, 64), dtype=np.float32)
    k[:, :, 5] += 25.0
    return xs, k


def canary_inputs():
    """Seeded canary inputs: (small q, small kref) and (config-shaped q f16, kref f32)."""
    rng = np.random.default_rng(6)
    q = rng.standard_normal((3, 5, 8, 64), dtype=np.float32) * 3
    kref = rng.standard_normal((3, 70, 2, 64), dtype=np.float32) * 3
    q2 = rng.standard_normal((4, 8, 32, 128), dtype=np.float32).astype(np.float16)
    kref2 = rng.standard_normal((4, 64, 8, 128), dtype=np.float32)
    kref2[..., [3, 77]] *= 10
    return (q, kref), (q2, kref2)


PREFILL_CHUNK = 16


def cfg1_prefill(s: Script):
    """Chunked-prefill case on a config-1 store: each sequence's last PREFILL_CHUNK
    tokens as queries (f32 [rows, 32, D]) over its whole context."""
    prefill, req_of, row = [], [], 0
    for r, n in enumerate(CFG1_LENS):
        prefill.append((row, row + PREFILL_CHUNK, n, 0))
        req_of.append(r)
        row += PREFILL_CHUNK
    q = np.random.default_rng(s.seed + 9).standard_normal((row, 32, s.d), dtype=np.float32)
    return prefill, req_of, q


def case_script(name, h, d, bs, mem, lens, plan, seed=0, kg=32, vg=32, dtype="f32", extra_blocks=3):
    """A store filled like the reference's decode-test fixture
    (``tests/echokv_vllm/test_decode_kernel.py:21-48``): sequences over a seeded
    block permutation, written block by block with sequences interleaved, block
    ``bi`` of sequence ``s`` opened at ``plan[(bi + s) % len(plan)]``; K channel 1
    carries a +30 outlier."""
    rng = np.random.default_rng(seed + 500)
    nbs = [-(-n // bs) for n in lens]
    num_blocks = sum(nbs) + extra_blocks
    perm = rng.permutation(num_blocks)
    table = np.zeros((len(lens), max(nbs)), np.int64)
    o = 0
    for i, nb in enumerate(nbs):
        table[i, :nb] = perm[o : o + nb]
        o += nb
    steps = []
    for bi in range(max(nbs)):
        for si, n in enumerate(lens):
            lo, hi = bi * bs, min((bi + 1) * bs, n)
            if lo >= hi:
                continue
            steps.append((table[si, bi] * bs + np.arange(hi - lo, dtype=np.int64), plan[(bi + si) % len(plan)]))
    s = Script(name, h, d, bs, mem, kg, vg, num_blocks, len(lens) + 2, steps, seed=seed, dtype=dtype,
               outliers=((1, 30.0),), full_bytes=False)
    s.meta = {"table": table, "lens": np.array(lens, np.int64)}
    return s


DECODE_CASES = [
    # name, h, d, bs, mem_bits, seq lens, tier plan, k_group
    ("dec_h2_d64_bs64", 2, 64, 64, 8, [1, 40, 64, 65, 200], [8, 4, 2], 32),
    ("dec_h1_d128_bs32_pool", 1, 128, 32, 4, [33, 97, 128], [8, 8, 4], 32),
    ("dec_h4_d64_mem6", 4, 64, 64, 6, [500, 3], [2, 4], 32),
    ("dec_h8_d128_bs64", 8, 128, 64, 8, [200, 70], [8, 4, 2], 32),
    ("dec_h8_d128_bs16_kg16", 8, 128, 16, 8, [300, 17, 1, 129], [4, 8, 2], 16),
]


def decode_case(i, seed=1, dtype="f32"):
    name, h, d, bs, mem, lens, plan, kg = DECODE_CASES[i]
    return case_script(f"{name}_s{seed}", h, d, bs, mem, lens, plan, seed=seed, kg=kg, dtype=dtype)
