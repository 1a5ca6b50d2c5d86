"""Write the golden fixtures under tests/golden/ from the reference implementation.

Run once, in the build container only (the reference tree exists nowhere
else):

    python tests/golden/make_golden.py [--reference /root/reference]

It imports the reference's ``echokv_vllm`` package (its PyTorch path, on the
CPU), replays every script of ``scripts.py`` through
``TieredKVCache``'s plan / prepare / commit / stage / apply sequence
(``echokv_vllm/tiered_cache.py:434-447``), and stores what the tests compare
against: the page bytes (whole pages for small scripts, per-page SHA-256 for
the config-1 stores), residual map, residual rows, K_ref ring, host counters,
each step's write plan, plus decode / prefill attention, canary and
quantization outputs. Only data is written; no reference source is copied.
With ``TRITON_INTERPRET=1`` set, the write kernels run in Triton's CPU
interpreter instead and the script records page hashes under ``triton_*``.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import scripts as S  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def run_script(s: S.Script, torch, tc, wp, dec, pf):
    layout = tc.TieredLayout(num_kv_heads=s.h, head_size=s.d, block_size=s.bs, mem_bits=s.mem_bits,
                             k_group=s.kg, v_group=s.vg)
    page = s.bs * tc.TieredLayout.per_token_bytes(s.h, s.d, s.mem_bits, s.kg, s.vg)
    stride = page + s.row_pad
    backing = torch.full((s.num_blocks * stride + 64,), 0xAB, dtype=torch.uint8)
    pages = torch.as_strided(backing, (s.num_blocks, page), (stride, 1))
    rdt = torch.float16 if s.dtype == "f16" else torch.float32
    store = tc.TieredKVCache(layout, pages, residual_slots=s.residual_slots, residual_dtype=rdt)
    kref = None
    if s.kref_window is not None:
        kref = torch.zeros(s.kref_window, s.h, s.d)
    plans = {}
    for i, (slots, bits, k, v) in enumerate(S.script_inputs(s)):
        kt, vt = torch.from_numpy(k), torch.from_numpy(v)
        plan = store.planner.plan(torch.from_numpy(slots))
        opened = store.prepare(plan, bits)
        store.shared.commit(plan)
        meta, extra = wp.stage_plan(plan, "cpu", opened)
        store.shared.apply_res_map(*extra[:4])
        if opened is not None:
            store.write_headers(extra[4], extra[5])
        store.apply(meta, kt, vt, kref)
        if s.full_bytes:
            plans[f"plan{i}_tok"] = np.stack([plan.tok_slot, plan.tok_res, plan.tok_sealed, plan.tok_kref])
            plans[f"plan{i}_fin"] = plan.fin
            plans[f"plan{i}_evict"] = np.array([[e.slot, e.block, e.group, e.fill] for e in plan.evictions],
                                               np.int64).reshape(-1, 4)
            hdr = np.zeros((0, 17), np.int64) if opened is None else np.concatenate(
                [opened[0][:, None], opened[1].astype(np.int64)], 1)
            plans[f"plan{i}_open"] = hdr
    out = dict(plans)
    pg = pages.numpy()
    out["page_sha"] = np.array([sha(pg[b]) for b in range(s.num_blocks)])
    out["pages_sha"] = np.array(sha(pg))
    if s.full_bytes:
        out["pages"] = pg.copy()
        out["guard_ok"] = np.array(all(
            bool((backing[b * stride + page : (b + 1) * stride] == 0xAB).all()) for b in range(s.num_blocks)))
    out["block_res"] = store.block_res.numpy().copy()
    out["res_group"] = store.res_group.numpy().copy()
    live = store.block_res[store.block_res >= 0]
    out["res_live_slots"] = live.numpy().copy()
    out["res_live"] = store.res_k[live].numpy().copy()
    if kref is not None:
        out["kref"] = kref.numpy().copy()
        out["kref_pos"] = np.array(store.planner.kref_pos)
        out["kref_fill"] = np.array(store.planner.kref_fill)
    tw = store.tokens_written
    out["counters"] = np.array([
        tw[2], tw[4], tw[8],
        store.blocks_opened[2], store.blocks_opened[4], store.blocks_opened[8],
        store.downgraded_blocks, store.demoted_blocks, store.sealed_groups,
        store.pool_free, store.residual_free,
    ], np.int64)
    out["tags"] = store.tag.numpy().copy()
    if s.name.startswith("cfg1"):
        table = torch.from_numpy(s.meta["table"]).to(torch.int32)
        lens = torch.from_numpy(s.meta["lens"])
        q = torch.from_numpy(S.cfg1_query(s))
        out["decode_out"] = dec.decode_attention_torch(store, q, table, lens, s.d ** -0.5).numpy()
        if s.name == "cfg1_int4_bs16":
            prefill, req_of, pq = S.cfg1_prefill(s)
            pq = torch.from_numpy(pq)
            pout = torch.zeros_like(pq)
            pf.prefill_attention_torch(store, pq, pout, prefill, table, s.d ** -0.5, req_of=req_of)
            out["prefill_out"] = pout.numpy()
            # Dequantized K/V of sequence 0's first 64 tokens (the read oracle, gather).
            pos = torch.arange(64)
            kk, vv = store.gather(table[0].long()[pos // s.bs], pos % s.bs)
            out["gather0_k"] = kk.numpy()
            out["gather0_v"] = vv.numpy()
    return out


def quant_fixture(torch, q):
    xs, k = S.quant_inputs()
    out = {}
    for shift, x in xs.items():
        for bits in (2, 4, 8):
            c, sc, mn = q.quantize(torch.from_numpy(x), bits, 32)
            tag = f"s{int(shift)}_b{bits}"
            out[f"codes_{tag}"] = c.numpy()
            out[f"scale_{tag}"] = sc.numpy()
            out[f"min_{tag}"] = mn.numpy()
            out[f"packed_{tag}"] = q.pack(c, bits).numpy()
    for bits in (2, 4, 8):
        out[f"fqc_b{bits}"] = q.fake_quant_channels(torch.from_numpy(k), bits, 32).numpy()
        sc, mn = q.stats_along(torch.from_numpy(k[:32]), bits, 0)
        out[f"stats_scale_b{bits}"] = sc.numpy()
        out[f"stats_min_b{bits}"] = mn.numpy()
    return out


def canary_fixture(torch, canary):
    (q, kref), (q2, kref2) = S.canary_inputs()
    out = {}
    out["small_out"] = canary.canary_kl(torch.from_numpy(q), torch.from_numpy(kref), (2, 4, 8), 32, 64 ** -0.5).numpy()
    out["cfg_out"] = canary.canary_kl(torch.from_numpy(q2), torch.from_numpy(kref2), (2, 4, 8), 16,
                                      128 ** -0.5).numpy()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--only", default=None)
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    import torch

    from echokv_vllm import canary, quant, tiered_cache as tc, write_plan as wp
    from echokv_vllm.kernels import decode as dec, prefill as pf

    triton = os.environ.get("TRITON_INTERPRET") == "1"
    manifest = {}
    for s in S.all_scripts():
        if args.only and args.only not in s.name:
            continue
        out = run_script(s, torch, tc, wp, dec, pf)
        if triton:
            manifest[s.name] = {"triton_pages_sha": str(out["pages_sha"])}
            continue
        np.savez_compressed(HERE / f"store_{s.name}.npz", **out)
        manifest[s.name] = {"pages_sha": str(out["pages_sha"])}
        print(s.name, manifest[s.name], flush=True)
    if triton:
        (HERE / "triton_interp_hashes.json").write_text(json.dumps(manifest, indent=1, sort_keys=True))
        print(json.dumps(manifest, indent=1))
        return
    if not args.only:
        np.savez_compressed(HERE / "quant.npz", **quant_fixture(torch, quant))
        np.savez_compressed(HERE / "canary.npz", **canary_fixture(torch, canary))
    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=1, sort_keys=True))


if __name__ == "__main__":
    main()
