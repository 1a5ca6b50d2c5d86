"""The reference's PyTorch path restated in torch on the CPU (TEST INFRASTRUCTURE:
the benchmark's CPU baseline; never imported by ``echokv_amd``).

Four legs, each a batched restatement over raw page bytes (a ``PageStore``'s
numpy arrays, shared with torch without a copy), pinned by ``tests/test_torch_cpu.py``
against the numpy oracle and the reference's golden bytes:

* decode: gather + dequantize + SDPA per sequence (``echokv_vllm/kernels/decode.py:95-129``
  over ``echokv_vllm/tiered_cache.py:451-478``);
* write: the step's token rows, then its completed K groups
  (``echokv_vllm/kernels/write.py:61-121``), in the order the store issues them
  (``tiered_cache.py:415-432``: finalize, then tokens);
* prefill: gather + SDPA with the bottom-right causal mask
  (``echokv_vllm/kernels/prefill.py:210-236``);
* canary: the batched per-tier attention KL (``echokv_vllm/canary.py:59-89``).

Numerics follow ``echokv_vllm/quant.py``: float32 extremes and IEEE division,
fp16-rounded stats, codes rounded half to even (``torch.round``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

TINY = 2.0 ** -14  # quant.py:23


def _levels(bits: int) -> float:
    return float((1 << bits) - 1)


# -- storage numerics (quant.py:26-120) ----------------------------------------
def quantize(x: torch.Tensor, bits: int, group: int):
    """quant.py:26-45: codes u8, scale / min fp16 per group of the last dim."""
    d = x.shape[-1]
    xg = x.float().reshape(*x.shape[:-1], d // group, group)
    mn16 = xg.amin(-1).half()
    mn = mn16.float()
    sc16 = ((xg.amax(-1) - mn) / _levels(bits)).clamp_min(TINY).half()
    q = torch.round((xg - mn[..., None]) / sc16.float()[..., None]).clamp(0, _levels(bits))
    return q.reshape(x.shape).to(torch.uint8), sc16, mn16


def stats_along(x: torch.Tensor, bits: int, dim: int):
    """quant.py:63-69."""
    xf = x.float()
    mn16 = xf.amin(dim).half()
    sc16 = ((xf.amax(dim) - mn16.float()) / _levels(bits)).clamp_min(TINY).half()
    return sc16, mn16


def quantize_with(x: torch.Tensor, sc16: torch.Tensor, mn16: torch.Tensor, bits: int) -> torch.Tensor:
    """quant.py:72-75."""
    q = torch.round((x.float() - mn16.float()) / sc16.float())
    return q.clamp(0, _levels(bits)).to(torch.uint8)


def pack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """quant.py:99-110: element i of a byte at bits [i*b, (i+1)*b)."""
    if bits == 8:
        return codes.to(torch.uint8)
    per = 8 // bits
    c = codes.reshape(*codes.shape[:-1], codes.shape[-1] // per, per).to(torch.int32)
    shifts = torch.arange(per, dtype=torch.int32) * bits
    return (c << shifts).sum(-1).to(torch.uint8)


def unpack(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """quant.py:113-120."""
    if bits == 8:
        return packed
    per = 8 // bits
    shifts = torch.arange(per, dtype=torch.int32) * bits
    c = (packed.to(torch.int32)[..., None] >> shifts) & ((1 << bits) - 1)
    return c.reshape(*packed.shape[:-1], packed.shape[-1] * per).to(torch.uint8)


# -- addressing (tiered_cache.py:120-147, 350-375) -------------------------------
class Pages:
    """Torch views of a ``PageStore`` (``oracle.store``): pages u8 [nb, page],
    residual, residual map. Writes land in the store's own arrays."""

    def __init__(self, ps):
        self.L = ps.L
        self.pages = torch.from_numpy(ps.pages)
        self.res_k = torch.from_numpy(ps.res_k)
        self.block_res = torch.from_numpy(ps.block_res)
        self.res_group = torch.from_numpy(ps.res_group)
        self.o = ps.L.offsets

    def tags(self, blk: torch.Tensor) -> torch.Tensor:
        return self.pages[blk, 0].to(torch.int64)

    def rows(self, blk: torch.Tensor, off: torch.Tensor, bits: int):
        """(page, byte) of each token's K+V row at ``bits`` (chunk 0 in the block's
        own page, chunk j >= 1 at pool chunk id table[j - 1] = page * KC + slot)."""
        L = self.L
        tpc = L.tokens_per_chunk(bits)
        j = off // tpc
        table = self.pages[blk, 4:16].contiguous().view(torch.int32).to(torch.int64)  # [n, 3]
        ids = table.gather(1, (j - 1).clamp_min(0)[:, None])[:, 0]
        page = torch.where(j > 0, ids // L.kc, blk)
        cslot = torch.where(j > 0, ids % L.kc, torch.zeros_like(ids))
        return page, self.o["data"] + cslot * L.chunk_bytes + (off % tpc) * 2 * L.side_bytes(bits)

    def f16(self, blk: torch.Tensor, start: torch.Tensor, count: int) -> torch.Tensor:
        cols = torch.arange(2 * count)
        return self.pages[blk[:, None], start[:, None] + cols].contiguous().view(torch.float16)

    def put(self, page: torch.Tensor, start: torch.Tensor, data: torch.Tensor) -> None:
        """Bytes ``data [n, w]`` at (page[i], start[i] + 0..w-1)."""
        cols = torch.arange(data.shape[1])
        self.pages[page[:, None], start[:, None] + cols] = data

    def put_f16(self, blk: torch.Tensor, start: torch.Tensor, x: torch.Tensor) -> None:
        self.put(blk, start, x.half().contiguous().view(torch.uint8).reshape(x.shape[0], -1))


# -- read: gather (tiered_cache.py:451-478) ----------------------------------------
def gather(P: Pages, blk: torch.Tensor, off: torch.Tensor):
    """Dequantized K, V float32 [n, H, D]; never-opened blocks read as zeros; a
    block's open K group reads the residual."""
    L, o = P.L, P.o
    n = blk.numel()
    k = torch.zeros(n, L.h, L.d)
    v = torch.zeros(n, L.h, L.d)
    tags = P.tags(blk)
    for bits in (2, 4, 8):
        m = torch.nonzero(tags == bits)[:, 0]
        if not m.numel():
            continue
        b, t = blk[m], off[m]
        page, byte = P.rows(b, t, bits)
        sb = L.side_bytes(bits)
        cols = torch.arange(sb)
        raw = P.pages[page[:, None], byte[:, None] + cols]
        kc = unpack(raw.reshape(-1, L.h, sb // L.h), bits).float()
        vc = unpack(P.pages[page[:, None], byte[:, None] + sb + cols].reshape(-1, L.h, sb // L.h), bits).float()
        ng, nk = L.h * L.g, L.h * L.d
        vs = P.f16(b, o["v_scale"] + t * ng * 2, ng).reshape(-1, L.h, L.g, 1).float()
        vm = P.f16(b, o["v_min"] + t * ng * 2, ng).reshape(-1, L.h, L.g, 1).float()
        g = t // L.kg
        ks = P.f16(b, o["k_scale"] + g * nk * 2, nk).reshape(-1, L.h, L.d).float()
        km = P.f16(b, o["k_min"] + g * nk * 2, nk).reshape(-1, L.h, L.d).float()
        v[m] = (vc.reshape(-1, L.h, L.g, L.vg) * vs + vm).reshape(-1, L.h, L.d)
        k[m] = kc * ks + km
    slot = P.block_res[blk]
    in_res = (slot >= 0) & (P.res_group[slot.clamp_min(0)] == off // L.kg) & ((tags == 2) | (tags == 4) | (tags == 8))
    r = torch.nonzero(in_res)[:, 0]
    if r.numel():
        k[r] = P.res_k[slot[r], off[r] % L.kg].float()
    return k, v


def _kv_of(P: Pages, table_row: torch.Tensor, n: int):
    pos = torch.arange(n)
    return gather(P, table_row[pos // P.L.bs], pos % P.L.bs)


def decode(ps, query: torch.Tensor, block_table, seq_lens, scale: float) -> torch.Tensor:
    """decode.py:95-129: ``query [S, Hq, D]`` -> float32 [S, Hq, D]."""
    P = Pages(ps)
    table = torch.as_tensor(block_table).to(torch.int64)
    out = torch.zeros(query.shape)
    for i, n in enumerate(torch.as_tensor(seq_lens).tolist()):
        if n <= 0:
            continue
        k, v = _kv_of(P, table[i], n)
        q = query[i].float()[:, None, :]  # [Hq, 1, D]
        out[i] = F.scaled_dot_product_attention(q, k.transpose(0, 1), v.transpose(0, 1), scale=scale,
                                                enable_gqa=True)[:, 0]
    return out


def prefill(ps, query: torch.Tensor, chunks, req_of, block_table, scale: float) -> torch.Tensor:
    """prefill.py:210-236: ``chunks`` = [(q_start, q_end, ctx, _)]; query i of a chunk of
    nq sees keys <= ctx - nq + i."""
    P = Pages(ps)
    table = torch.as_tensor(block_table).to(torch.int64)
    out = torch.zeros(query.shape)
    for (qs, qe, ctx, _), r in zip(chunks, req_of):
        nq = qe - qs
        k, v = _kv_of(P, table[r], ctx)
        keep = torch.arange(ctx)[None, :] <= (ctx - nq + torch.arange(nq))[:, None]
        q = query[qs:qe].float().transpose(0, 1)  # [Hq, nq, D]
        out[qs:qe] = F.scaled_dot_product_attention(q, k.transpose(0, 1), v.transpose(0, 1), attn_mask=keep,
                                                    scale=scale, enable_gqa=True).transpose(0, 1)
    return out


# -- write (write.py:61-121) -----------------------------------------------------------
def _write_side(P: Pages, blk, off, bits, codes, side):
    page, byte = P.rows(blk, off, bits)
    sb = P.L.side_bytes(bits)
    P.put(page, byte + side * sb, pack(codes, bits).reshape(codes.shape[0], -1))


def finalize_k(ps, key: torch.Tensor, fin) -> None:
    """write.py:96-121: fin rows [block, group, residual slot, token row per position]."""
    P, L = Pages(ps), ps.L
    fin = torch.as_tensor(fin).to(torch.int64).reshape(-1, 3 + L.kg)
    if not fin.shape[0]:
        return
    blk, grp, rs, rows = fin[:, 0], fin[:, 1], fin[:, 2].clamp_min(0), fin[:, 3:]
    x = torch.where((rows >= 0)[..., None, None], key.float()[rows.clamp_min(0)], P.res_k[rs].float())  # [f, KG, H, D]
    tags = P.tags(blk)
    nk = L.h * L.d
    for bits in (2, 4, 8):
        m = torch.nonzero(torch.where(tags == 0, 2, tags) == bits)[:, 0]
        if not m.numel():
            continue
        sc, mn = stats_along(x[m], bits, 1)  # [f, H, D]
        start = P.o["k_scale"] + grp[m] * nk * 2
        P.put_f16(blk[m], start, sc.reshape(m.numel(), -1))
        P.put_f16(blk[m], P.o["k_min"] + grp[m] * nk * 2, mn.reshape(m.numel(), -1))
        codes = quantize_with(x[m], sc[:, None], mn[:, None], bits)  # [f, KG, H, D]
        tb = blk[m].repeat_interleave(L.kg)
        to = (grp[m][:, None] * L.kg + torch.arange(L.kg)).reshape(-1)
        _write_side(P, tb, to, bits, codes.reshape(-1, L.h, L.d), 0)


def write_tokens(ps, key: torch.Tensor, value: torch.Tensor, tok, kref: torch.Tensor | None = None) -> None:
    """write.py:61-95: ``tok [4, n]`` = (slot, residual slot, sealed, K_ref row)."""
    P, L = Pages(ps), ps.L
    tok = torch.as_tensor(tok).to(torch.int64)
    live = torch.nonzero(tok[0] >= 0)[:, 0]
    if not live.numel():
        return
    slot, rslot, sealed, kidx = tok[0, live], tok[1, live], tok[2, live], tok[3, live]
    blk, off = slot // L.bs, slot % L.bs
    tags = P.tags(blk)
    kx, vx = key.float()[live], value.float()[live]
    ng = L.h * L.g
    for bits in (2, 4, 8):
        m = torch.nonzero(torch.where(tags == 0, 2, tags) == bits)[:, 0]
        if not m.numel():
            continue
        codes, sc, mn = quantize(vx[m], bits, L.vg)
        P.put_f16(blk[m], P.o["v_scale"] + off[m] * ng * 2, sc.reshape(m.numel(), -1))
        P.put_f16(blk[m], P.o["v_min"] + off[m] * ng * 2, mn.reshape(m.numel(), -1))
        _write_side(P, blk[m], off[m], bits, codes, 1)
        s = m[sealed[m] != 0]
        if s.numel():  # K under the group's stored stats
            g = off[s] // L.kg
            nk = L.h * L.d
            ks = P.f16(blk[s], P.o["k_scale"] + g * nk * 2, nk).reshape(-1, L.h, L.d)
            km = P.f16(blk[s], P.o["k_min"] + g * nk * 2, nk).reshape(-1, L.h, L.d)
            _write_side(P, blk[s], off[s], bits, quantize_with(kx[s], ks, km, bits), 0)
    r = torch.nonzero(rslot >= 0)[:, 0]
    if r.numel():
        P.res_k[rslot[r], off[r] % L.kg] = kx[r].to(P.res_k.dtype)
    if kref is not None:
        kr = torch.nonzero(kidx >= 0)[:, 0]
        if kr.numel():
            kref[kidx[kr]] = kx[kr].to(kref.dtype)


def write_step(ps, key: torch.Tensor, value: torch.Tensor, tok, fin, kref=None) -> None:
    """One step's writes as the store issues them (tiered_cache.py:425-432)."""
    finalize_k(ps, key, fin)
    write_tokens(ps, key, value, tok, kref)


# -- canary (canary.py:59-89) --------------------------------------------------------
def fake_quant_channels(k: torch.Tensor, bits: int, group: int) -> torch.Tensor:
    """quant.py:82-96 over ``k [..., T, H, D]``; a trailing partial group stays exact."""
    t = k.shape[-3]
    full = (t // group) * group
    out = k.float().clone()
    if full:
        kg = out[..., :full, :, :].reshape(*k.shape[:-3], full // group, group, *k.shape[-2:])
        sc, mn = stats_along(kg, bits, -3)
        q = quantize_with(kg, sc[..., None, :, :], mn[..., None, :, :], bits).float()
        deq = q * sc.float()[..., None, :, :] + mn.float()[..., None, :, :]
        out[..., :full, :, :] = deq.reshape(*k.shape[:-3], full, *k.shape[-2:])
    return out


def canary_kl(query: torch.Tensor, kref: torch.Tensor, bits, k_group: int, scale: float) -> torch.Tensor:
    """query [..., nq, Hq, D], kref [..., W, H, D] (oldest first) -> [..., len(bits)]."""
    w = (kref.shape[-3] // k_group) * k_group
    kref = kref[..., kref.shape[-3] - w :, :, :].float()
    q = query.float().transpose(-3, -2)  # [..., Hq, nq, D]
    rep = q.shape[-3] // kref.shape[-2]

    def logw(k):
        kh = k.transpose(-3, -2).repeat_interleave(rep, dim=-3)  # [..., Hq, W, D]
        return torch.log_softmax(q @ kh.transpose(-1, -2) * scale, dim=-1)

    lref = logw(kref)
    out = []
    for b in bits:
        lq = logw(fake_quant_channels(kref, b, k_group))
        out.append((lq.exp() * (lq - lref)).sum(-1).mean(dim=(-2, -1)))
    return torch.stack(out, -1).clamp_min(0.0)
