"""Paged tiered store in numpy (oracle; test infrastructure only).

Restates the device-side effects of the reference store on raw page bytes:

* layout and addressing: ``echokv_vllm/tiered_cache.py:99-147`` (offsets),
  ``tiered_cache.py:350-375`` (chunk / row / byte of a token, pack into a side);
* token writes: ``echokv_vllm/kernels/write.py:61-95`` (V per token, K to the
  residual or under sealed stats, K_ref ring);
* K-group finalize: ``write.py:96-121``;
* seal of an evicted residual group: ``tiered_cache.py:379-394``;
* LRU demotion requantization to INT2: ``tiered_cache.py:322-340``;
* ``gather`` (the read oracle): ``tiered_cache.py:451-478``.

Host decisions (which blocks open, chunk ids, residual slots) are not here:
the tests drive these functions with the product's host planner.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import quant as Q


@dataclass(frozen=True)
class Layout:
    """``TieredLayout`` offsets (``tiered_cache.py:120-147``)."""

    h: int
    d: int
    bs: int
    mem_bits: int
    kg: int = 32
    vg: int = 32

    @property
    def kgb(self):
        return self.bs // self.kg

    @property
    def g(self):
        return self.d // self.vg

    @property
    def kc(self):
        return self.mem_bits // 2

    @property
    def chunk_bytes(self):
        return self.bs * self.h * self.d // 2

    @property
    def offsets(self):
        bs, h, d = self.bs, self.h, self.d
        o = {"v_scale": bs}
        o["v_min"] = o["v_scale"] + bs * h * self.g * 2
        o["k_scale"] = o["v_min"] + bs * h * self.g * 2
        o["k_min"] = o["k_scale"] + self.kgb * h * d * 2
        o["data"] = o["k_min"] + self.kgb * h * d * 2
        o["end"] = o["data"] + self.kc * self.chunk_bytes
        return o

    def side_bytes(self, bits):
        return self.h * self.d * bits // 8

    def tokens_per_chunk(self, bits):
        return 2 * self.bs // bits


def per_token_bytes(h, d, mem_bits, kg=32, vg=32):
    """tiered_cache.py:99-106."""
    raw = 1 + 4 * h * (d // vg) + 4 * h * d // kg + (mem_bits // 2) * h * d // 2
    return -(-raw // 4) * 4


class PageStore:
    """One layer's pages (uint8 ``[num_blocks, page_bytes]``) plus the residual,
    residual map and K_ref ring, as numpy arrays."""

    def __init__(self, L: Layout, num_blocks: int, residual_slots: int, res_dtype=np.float32, page_bytes=None):
        self.L = L
        self.n = num_blocks
        self.page_bytes = page_bytes or L.bs * per_token_bytes(L.h, L.d, L.mem_bits, L.kg, L.vg)
        self.pages = np.zeros((num_blocks, self.page_bytes), np.uint8)
        self.res_k = np.zeros((residual_slots + 1, L.kg, L.h, L.d), res_dtype)
        self.block_res = np.full(num_blocks, -1, np.int64)
        self.res_group = np.zeros(residual_slots + 1, np.int64)

    @classmethod
    def over(cls, L: Layout, pages, res_k, block_res, res_group):
        """A store over existing arrays (e.g. a device store's bytes copied to the host)."""
        ps = cls.__new__(cls)
        ps.L, ps.n = L, pages.shape[0]
        ps.page_bytes = pages.shape[1]
        ps.pages = pages
        ps.res_k = res_k
        ps.block_res = np.asarray(block_res, np.int64)
        ps.res_group = np.asarray(res_group, np.int64)
        return ps

    # -- typed views ------------------------------------------------------
    def _f16(self, blk, start, count):
        return self.pages[blk, start : start + 2 * count].view(np.float16)

    def tag(self, blk):
        return int(self.pages[blk, 0])

    def table(self, blk):
        return self.pages[blk, 4:16].view(np.int32)

    def v_stats(self, blk, off):
        """(scale, min) fp16 ``[H, G]`` views of token ``off`` (tiered_cache.py:189-190)."""
        L, o = self.L, self.L.offsets
        n = L.h * L.g
        s = self._f16(blk, o["v_scale"] + off * n * 2, n).reshape(L.h, L.g)
        m = self._f16(blk, o["v_min"] + off * n * 2, n).reshape(L.h, L.g)
        return s, m

    def k_stats(self, blk, grp):
        """(scale, min) fp16 ``[H, D]`` views of K group ``grp`` (tiered_cache.py:191-192)."""
        L, o = self.L, self.L.offsets
        n = L.h * L.d
        s = self._f16(blk, o["k_scale"] + grp * n * 2, n).reshape(L.h, L.d)
        m = self._f16(blk, o["k_min"] + grp * n * 2, n).reshape(L.h, L.d)
        return s, m

    # -- addressing (tiered_cache.py:350-375; write.py:142-153) -------------
    def locate(self, blk: int, off: int, bits: int):
        """(page, byte offset inside the page) of token ``off``'s K+V row at ``bits``."""
        L = self.L
        tpc = L.tokens_per_chunk(bits)
        j = off // tpc
        if j > 0:
            cid = int(self.table(blk)[j - 1])
            page, slot = cid // L.kc, cid % L.kc
        else:
            page, slot = blk, 0
        return page, L.offsets["data"] + slot * L.chunk_bytes + (off % tpc) * 2 * L.side_bytes(bits)

    def write_side(self, blk, off, bits, codes, side):
        """Pack ``codes [H, D]`` into the K (side 0) or V (side 1) half of a row."""
        page, byte = self.locate(blk, off, bits)
        sb = self.L.side_bytes(bits)
        self.pages[page, byte + side * sb : byte + (side + 1) * sb] = Q.pack(codes, bits).reshape(-1)

    def read_side(self, blk, off, bits, side):
        page, byte = self.locate(blk, off, bits)
        sb = self.L.side_bytes(bits)
        return Q.unpack(self.pages[page, byte + side * sb : byte + (side + 1) * sb].reshape(self.L.h, -1), bits)

    @staticmethod
    def _bits(tag):
        return 2 if tag == 0 else tag  # common.py:32-34, write.py:192,250

    # -- device effects of a step ----------------------------------------
    def write_headers(self, blocks, headers):
        """tiered_cache.py:305-307."""
        for b, hdr in zip(np.asarray(blocks).tolist(), np.asarray(headers, np.uint8)):
            self.pages[b, :16] = hdr

    def apply_res_map(self, blocks, values, slots, groups):
        """write_plan.py:266-271."""
        self.block_res[np.asarray(blocks, np.int64)] = values
        self.res_group[np.asarray(slots, np.int64)] = groups

    def write_tokens(self, key, value, tok, kref=None):
        """write.py:61-95 (and the Triton kernel write.py:172-229): ``tok [4, n]``."""
        L = self.L
        for t in range(tok.shape[1]):
            slot = int(tok[0, t])
            if slot < 0:
                continue
            blk, off = slot // L.bs, slot % L.bs
            bits = self._bits(self.tag(blk))
            codes, sc, mn = Q.quantize(value[t], bits, L.vg)
            s, m = self.v_stats(blk, off)
            s[...] = sc
            m[...] = mn
            self.write_side(blk, off, bits, codes, 1)
            kx = key[t]
            r = int(tok[1, t])
            if r >= 0:
                self.res_k[r, off % L.kg] = kx.astype(self.res_k.dtype)
            if int(tok[2, t]) != 0:
                ks, km = self.k_stats(blk, off // L.kg)
                self.write_side(blk, off, bits, Q.quantize_with(kx, ks, km, bits), 0)
            if kref is not None and int(tok[3, t]) >= 0:
                kref[int(tok[3, t])] = kx.astype(kref.dtype)

    def finalize_k(self, key, fin):
        """write.py:96-121 (Triton write.py:232-287): one row per completed K group."""
        L = self.L
        for row in np.asarray(fin, np.int64):
            blk, grp, rs = int(row[0]), int(row[1]), int(row[2])
            rows = row[3:]
            x = np.empty((L.kg, L.h, L.d), np.float32)
            for p in range(L.kg):
                x[p] = key[rows[p]].astype(np.float32) if rows[p] >= 0 else self.res_k[max(rs, 0), p].astype(np.float32)
            bits = self._bits(self.tag(blk))
            sc, mn = Q.stats_along(x, bits, 0)
            ks, km = self.k_stats(blk, grp)
            ks[...] = sc
            km[...] = mn
            codes = Q.quantize_with(x, sc, mn, bits)
            for p in range(L.kg):
                self.write_side(blk, grp * L.kg + p, bits, codes[p], 0)

    def seal(self, slot, block, group, fill, bits, mask):
        """tiered_cache.py:379-394: quantize an evicted group's ``fill`` tokens under their own stats."""
        if fill <= 0:
            return
        ks = self.res_k[slot, :fill].astype(np.float32)
        sc, mn = Q.stats_along(ks, bits, 0)
        s, m = self.k_stats(block, group)
        s[...] = sc
        m[...] = mn
        codes = Q.quantize_with(ks, sc, mn, bits)
        for p in range(fill):
            self.write_side(block, group * self.L.kg + p, bits, codes[p], 0)
        self.pages[block, 1] = mask

    def demote(self, victims):
        """tiered_cache.py:322-340: requantize whole blocks to INT2 in place (K per channel
        over K groups, V per token); read at the current tiers first."""
        L = self.L
        if not len(victims):
            return
        vb = np.asarray(victims, np.int64)
        blk = np.repeat(vb, L.bs)
        off = np.tile(np.arange(L.bs), vb.size)
        k, v = self.gather(blk, off)
        kg = k.reshape(vb.size, L.kgb, L.kg, L.h, L.d)
        ksc, kmn = Q.stats_along(kg, 2, 2)
        kcodes = Q.quantize_with(kg, ksc[:, :, None], kmn[:, :, None], 2).reshape(-1, L.h, L.d)
        vcodes, vsc, vmn = Q.quantize(v, 2, L.vg)
        for i, b in enumerate(vb.tolist()):
            self.pages[b, 0] = 2
            for g in range(L.kgb):
                s, m = self.k_stats(b, g)
                s[...] = ksc[i, g]
                m[...] = kmn[i, g]
        for i in range(blk.size):
            b, o = int(blk[i]), int(off[i])
            s, m = self.v_stats(b, o)
            s[...] = vsc[i]
            m[...] = vmn[i]
            self.write_side(b, o, 2, kcodes[i], 0)
            self.write_side(b, o, 2, vcodes[i], 1)

    # -- read ---------------------------------------------------------------
    def gather(self, blk, off):
        """tiered_cache.py:451-478: dequantized K, V float32 ``[n, H, D]``; the block's
        open K group reads the residual."""
        L = self.L
        blk = np.asarray(blk, np.int64).reshape(-1)
        off = np.asarray(off, np.int64).reshape(-1)
        n = blk.size
        k_out = np.zeros((n, L.h, L.d), np.float32)
        v_out = np.zeros((n, L.h, L.d), np.float32)
        for i in range(n):
            b, o = int(blk[i]), int(off[i])
            tag = self.tag(b)
            if tag not in Q.SUPPORTED_BITS:
                continue  # never opened: gather leaves zeros
            vc = self.read_side(b, o, tag, 1)
            s, m = self.v_stats(b, o)
            v_out[i] = Q.dequantize(vc, s, m, L.vg)
            slot = int(self.block_res[b])
            if slot >= 0 and int(self.res_group[slot]) == o // L.kg:
                k_out[i] = self.res_k[slot, o % L.kg].astype(np.float32)
            else:
                kc = self.read_side(b, o, tag, 0)
                ks, km = self.k_stats(b, o // L.kg)
                k_out[i] = Q.dequantize_with(kc, ks, km)
        return k_out, v_out

    def gather_seq(self, table_row, n):
        """K, V ``[n, H, D]`` of one sequence's first ``n`` tokens through its block-table row."""
        pos = np.arange(n)
        return self.gather(np.asarray(table_row, np.int64)[pos // self.L.bs], pos % self.L.bs)

    def raw_vec(self, blk, off, bits):
        """Stored codes and stats of tokens (blk, off) whose blocks are all at ``bits``,
        vectorized: K codes, V codes ``[n, H, D]`` u8; V scale / min ``[n, H, G]`` and
        K scale / min of each token's K group ``[n, H, D]`` fp16 (tiered_cache.py:350-375)."""
        L, o = self.L, self.L.offsets
        b = np.asarray(blk, np.int64).reshape(-1)
        t = np.asarray(off, np.int64).reshape(-1)
        n = b.size
        tpc = L.tokens_per_chunk(bits)
        j = t // tpc
        ids = self.pages[b, 4:16].copy().view(np.int32)[np.arange(n), np.maximum(j - 1, 0)].astype(np.int64)
        page = np.where(j > 0, ids // L.kc, b)
        cslot = np.where(j > 0, ids % L.kc, 0)
        sb = L.side_bytes(bits)
        base = o["data"] + cslot * L.chunk_bytes + (t % tpc) * 2 * sb
        cols = np.arange(sb)
        kc = Q.unpack(self.pages[page[:, None], base[:, None] + cols].reshape(n, L.h, -1), bits)
        vc = Q.unpack(self.pages[page[:, None], base[:, None] + sb + cols].reshape(n, L.h, -1), bits)
        ng, nk = L.h * L.g, L.h * L.d
        def f16(start, count):
            return self.pages[b[:, None], start[:, None] + np.arange(2 * count)].copy().view(np.float16)
        vs = f16(o["v_scale"] + t * ng * 2, ng).reshape(n, L.h, L.g)
        vm = f16(o["v_min"] + t * ng * 2, ng).reshape(n, L.h, L.g)
        g = t // L.kg
        ks = f16(o["k_scale"] + g * nk * 2, nk).reshape(n, L.h, L.d)
        km = f16(o["k_min"] + g * nk * 2, nk).reshape(n, L.h, L.d)
        return kc, vc, vs, vm, ks, km

    def gather_vec(self, blk, off):
        """``gather`` vectorized over tokens (numpy fancy indexing per tier); the same
        values, used where the per-token loop is too slow (the CPU baseline, tests at
        the benchmark configurations)."""
        L = self.L
        blk = np.asarray(blk, np.int64).reshape(-1)
        off = np.asarray(off, np.int64).reshape(-1)
        n = blk.size
        k_out = np.zeros((n, L.h, L.d), np.float32)
        v_out = np.zeros((n, L.h, L.d), np.float32)
        tags = self.pages[blk, 0].astype(np.int64)
        slot = self.block_res[blk]
        in_res = (slot >= 0) & (self.res_group[np.maximum(slot, 0)] == off // L.kg)
        for bits in Q.SUPPORTED_BITS:
            m = np.flatnonzero(tags == bits)
            if not m.size:
                continue
            kc, vc, vs, vm, ks, km = self.raw_vec(blk[m], off[m], bits)
            v_out[m] = Q.dequantize(vc, vs, vm, L.vg)
            k_out[m] = Q.dequantize_with(kc, ks, km)
        r = np.flatnonzero(in_res & np.isin(tags, Q.SUPPORTED_BITS))
        if r.size:
            k_out[r] = self.res_k[slot[r], off[r] % L.kg].astype(np.float32)
        return k_out, v_out
