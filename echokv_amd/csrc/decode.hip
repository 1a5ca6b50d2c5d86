// Split-KV paged decode attention over the tiered (INT2/INT4/INT8) pages, gfx950.
//
// Work decomposition: one workgroup per (sequence, split, group of <= 8 KV
// heads), one 64-wide wave per KV head. The heads of a token row sit side by
// side in a page ([K codes of all heads | V codes of all heads]), so the waves
// of a workgroup read neighbouring slices of the same cache lines together.
//
// Per 16-token tile a wave runs two MFMA contractions with no transposes:
//   S^T[t, q]  = sum_d codes[t, d] * (q[q, d] * k_scale[d]) + sum_d q[q, d] * k_min[d]
//                (v_mfma_f32_16x16x32_f16; the K scale is folded into the query,
//                 the K min into a per-query float32 bias; the block's open K
//                 group reads the full-precision residual instead)
//   O^T[d, q] += V[t, d]^T * P^T[t, q]   (v_mfma_f32_16x16x16f16, V dequantized
//                 to fp16 in registers with its per-token fp16 scale / min)
// Codes are exact in fp16. The query-side operand (q * k_scale, and the residual
// keys) is carried as an fp16 hi + lo pair -- lo = fma(q, s, -hi) rounded once --
// and contracted twice, so S is accurate to ~2^-22 instead of fp16's 2^-11:
// keys with large outlier channels would otherwise dominate the error.
// The S^T accumulator layout (lane = 4 tokens x 1 query column) is exactly the
// B-operand layout of the second MFMA, and the O^T accumulator keeps one query
// column per lane, so the online softmax runs per lane with two cross-lane
// max reductions per tile. Query columns are the GQA heads of the KV head,
// padded to 16. Codes become fp16 by OR-ing them under the exponent of 1024
// (0x6400) and subtracting 1024 (exact).
//
// A split covers max(blocks_per_split, ceil(blocks / num_splits)) blocks of
// the sequence's own length, so results do not depend on the rest of the
// batch; a second kernel merges the splits in order (log-sum-exp).
#include "args.h"

namespace ek {

__device__ __forceinline__ h2_t u2h(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t h2u(h2_t h) { return __builtin_bit_cast(uint32_t, h); }

// 0x6400 = fp16 1024.0; (1024 + c) - 1024 is exact for codes c < 1024.
__device__ __forceinline__ h2_t code_pair(uint32_t bits16x2) {
  const h2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  return u2h(bits16x2 | 0x64006400u) - k1024;
}

__device__ __forceinline__ h8_t cat8(h2_t a, h2_t b, h2_t c, h2_t d) {
  return h8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Eight channels (e0..e7, natural order) of a K row as an MFMA fragment in the
// tier's pair order: INT4 / INT2 give (e0,e4),(e1,e5),(e2,e6),(e3,e7); INT8 gives
// (e0,e2),(e1,e3),(e4,e6),(e5,e7). The query side uses the same order.
template <int BITS>
__device__ __forceinline__ h8_t unpack8(const uint32_t* w) {
  if constexpr (BITS == 4) {
    const uint32_t x = w[0];
    return cat8(code_pair(x & 0x000F000Fu), code_pair((x >> 4) & 0x000F000Fu), code_pair((x >> 8) & 0x000F000Fu),
                code_pair((x >> 12) & 0x000F000Fu));
  } else if constexpr (BITS == 8) {
    const uint32_t x = w[0], y = w[1];
    return cat8(code_pair(x & 0x00FF00FFu), code_pair((x >> 8) & 0x00FF00FFu), code_pair(y & 0x00FF00FFu),
                code_pair((y >> 8) & 0x00FF00FFu));
  } else {
    const uint32_t u = w[0] & 0xFFFFu;
    const uint32_t x = (u & 0xFFu) | ((u & 0xFF00u) << 8);
    return cat8(code_pair(x & 0x00030003u), code_pair((x >> 2) & 0x00030003u), code_pair((x >> 4) & 0x00030003u),
                code_pair((x >> 6) & 0x00030003u));
  }
}

// Natural pairs n[0..3] = (e0,e1),(e2,e3),(e4,e5),(e6,e7) -> the tier's order.
template <int BITS>
__device__ __forceinline__ h8_t reorder8(const uint32_t* n) {
  if constexpr (BITS == 8) {
    return cat8(u2h(__builtin_amdgcn_perm(n[1], n[0], 0x05040100u)), u2h(__builtin_amdgcn_perm(n[1], n[0], 0x07060302u)),
                u2h(__builtin_amdgcn_perm(n[3], n[2], 0x05040100u)), u2h(__builtin_amdgcn_perm(n[3], n[2], 0x07060302u)));
  } else {
    return cat8(u2h(__builtin_amdgcn_perm(n[2], n[0], 0x05040100u)), u2h(__builtin_amdgcn_perm(n[2], n[0], 0x07060302u)),
                u2h(__builtin_amdgcn_perm(n[3], n[1], 0x05040100u)), u2h(__builtin_amdgcn_perm(n[3], n[1], 0x07060302u)));
  }
}

// Load `NB` bytes (1, 2, 4, 8, 16 or 32) at p into 32-bit words.
template <int NB>
__device__ __forceinline__ void load_bytes(const uint8_t* p, uint32_t* w) {
  if constexpr (NB == 1) {
    w[0] = *p;
  } else if constexpr (NB == 2) {
    w[0] = *(const uint16_t*)p;
  } else if constexpr (NB == 4) {
    w[0] = *(const uint32_t*)p;
  } else if constexpr (NB == 8) {
    const uint2 x = *(const uint2*)p;
    w[0] = x.x;
    w[1] = x.y;
  } else {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const uint4 x = ((const uint4*)p)[i];
      w[4 * i] = x.x;
      w[4 * i + 1] = x.y;
      w[4 * i + 2] = x.z;
      w[4 * i + 3] = x.w;
    }
  }
}

// Per-wave decode state for head_dim D. QLO: the query has a low part (float32 input).
template <int D, bool QLO>
struct Wave {
  static constexpr int CPL = D / 4;   // K channels per lane in the QK fragments
  static constexpr int NQK = D / 32;  // 16x16x32 MFMAs per tile for S^T (per hi / lo part)
  static constexpr int CPM = D / 16;  // V channels per lane = 16x16x16 MFMAs per tile
  uint32_t qn[CPL / 2];               // fp16 query pairs (hi), natural channel order
  uint32_t ql[QLO ? CPL / 2 : 1];     // fp16 query pairs (lo = q - hi)
  h8_t qk[NQK], qkl[NQK];             // q * k_scale (hi, lo) fragments, current K group
  float bias;                         // sum_d q * k_min for the current K group
  f4_t acc[CPM];                      // O^T fragments
  float m_run, l_lane;
};

// q * k_scale (hi / lo) fragments and the k_min bias of one K group, from the
// lane's CPL channels of k_scale at ksp and of k_min at kmp (global or LDS).
// Lanes of padding query columns (`active` false) hold zeros and skip the reads.
template <int D, bool QLO, int BITS>
__device__ __forceinline__ void build_qk_at(Wave<D, QLO>& w, const uint8_t* ksp, const uint8_t* kmp, bool active) {
  constexpr int CPL = Wave<D, QLO>::CPL;
  uint32_t ks[CPL / 2], km[CPL / 2];
  if (active) {
    load_bytes<2 * CPL>(ksp, ks);
    load_bytes<2 * CPL>(kmp, km);
  } else {
#pragma unroll
    for (int i = 0; i < CPL / 2; ++i) ks[i] = km[i] = 0;
  }
  float b = 0.f;
  uint32_t hi[CPL / 2], lo[CPL / 2];
#pragma unroll
  for (int i = 0; i < CPL / 2; ++i) {
    const h2_t q = u2h(w.qn[i]), s = u2h(ks[i]);
    const h2_t ph = q * s;
    h2_t pl = __builtin_elementwise_fma(q, s, -ph);  // exact product minus its rounding, rounded once
    b = __builtin_amdgcn_fdot2(q, u2h(km[i]), b, false);
    if constexpr (QLO) {
      pl = __builtin_elementwise_fma(u2h(w.ql[i]), s, pl);
      b = __builtin_amdgcn_fdot2(u2h(w.ql[i]), u2h(km[i]), b, false);
    }
    hi[i] = h2u(ph);
    lo[i] = h2u(pl);
  }
#pragma unroll
  for (int j = 0; j < Wave<D, QLO>::NQK; ++j) {
    w.qk[j] = reorder8<BITS>(hi + 4 * j);
    w.qkl[j] = reorder8<BITS>(lo + 4 * j);
  }
  b += __shfl_xor(b, 16, 64);
  b += __shfl_xor(b, 32, 64);
  w.bias = b;
}

template <int D, bool QLO, int BITS>
__device__ __forceinline__ void build_qk(Wave<D, QLO>& w, const uint8_t* pages, const Lay& L, long blk, int grp,
                                         int h, int c, bool active) {
  const long e0 = ((long)grp * L.H + h) * D + c * Wave<D, QLO>::CPL;
  build_qk_at<D, QLO, BITS>(w, pages + blk * L.stride + L.o_ks + 2 * e0, pages + blk * L.stride + L.o_km + 2 * e0,
                            active);
}

// Online-softmax update with the tile's S^T fragment (already scaled to log2
// units and masked), then O^T += V^T P^T.
template <int D, bool QLO>
__device__ __forceinline__ void softmax_pv(Wave<D, QLO>& w, f4_t s, const h4_t* va) {
  float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
  mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
  const float m_new = fmaxf(w.m_run, mt);
  const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_new);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(s[i] - m_new);
  w.l_lane = w.l_lane * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
  w.m_run = m_new;
  const h4_t pb = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
#pragma unroll
  for (int j = 0; j < Wave<D, QLO>::CPM; ++j) {
    w.acc[j] *= alpha;
    w.acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va[j], pb, w.acc[j], 0, 0, 0);
  }
}

// One 16-token tile [t0, t0 + 16) of block `blk` (tier BITS); tokens >= n_valid
// are masked. in_res: the tile is the block's open K group (K from the residual).
template <int D, bool QLO, int BITS>
__device__ __forceinline__ void tile(Wave<D, QLO>& w, const DecodeArgs& a, long blk, int t0, int n_valid, long rslot,
                                     bool in_res, int h, int lane) {
  using W = Wave<D, QLO>;
  constexpr int CPL = W::CPL, NQK = W::NQK, CPM = W::CPM;
  const Lay& L = a.L;
  const int c = lane >> 4, n = lane & 15;
  const uint8_t* pages = a.pages;
  const long side = (long)L.H * D * BITS / 8;
  const long headb = (long)h * (D * BITS / 8);

  // ---- S^T = K Q'^T (+ bias) -------------------------------------------
  f4_t s = {0.f, 0.f, 0.f, 0.f};
  const int tk = t0 + n;
  const bool kvalid = tk < n_valid;
  if (in_res) {
    const long r0 = rslot * a.res.s0 + (long)(tk % L.KG) * a.res.s1 + h * a.res.s2 + c * CPL;
    const bool res_lo = a.res.dtype == ECHOKV_F32;  // fp16 / bf16 keys are exact in fp16
    float xr[CPL];
    if (kvalid) {
      ld_n<CPL>(a.res.ptr, a.res.dtype, r0, xr);
    } else {
#pragma unroll
      for (int e = 0; e < CPL; ++e) xr[e] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      h8_t kh, kl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = xr[8 * j + e];
        kh[e] = (_Float16)x;
        kl[e] = (_Float16)(x - (float)kh[e]);
      }
      const h8_t qh = cat8(u2h(w.qn[4 * j]), u2h(w.qn[4 * j + 1]), u2h(w.qn[4 * j + 2]), u2h(w.qn[4 * j + 3]));
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh, s, 0, 0, 0);
      if (res_lo) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh, s, 0, 0, 0);
      if constexpr (QLO) {
        const h8_t ql = cat8(u2h(w.ql[4 * j]), u2h(w.ql[4 * j + 1]), u2h(w.ql[4 * j + 2]), u2h(w.ql[4 * j + 3]));
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql, s, 0, 0, 0);
      }
    }
  } else {
    const long rb = row_base(pages, L, blk, tk, BITS);
    constexpr int KW = CPL * BITS / 32 > 0 ? CPL * BITS / 32 : 1;
    uint32_t kw[KW];
    if (rb >= 0) {
      load_bytes<CPL * BITS / 8>(pages + rb + headb + (long)c * (CPL * BITS / 8), kw);
    } else {
#pragma unroll
      for (int i = 0; i < KW; ++i) kw[i] = 0;
    }
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      // 8 channels = BITS bytes of the lane's slice.
      uint32_t wj[2];
      if constexpr (BITS == 8) {
        wj[0] = kw[2 * j];
        wj[1] = kw[2 * j + 1];
      } else if constexpr (BITS == 4) {
        wj[0] = kw[j];
      } else {
        wj[0] = kw[j >> 1] >> (16 * (j & 1));
      }
      const h8_t kf = unpack8<BITS>(wj);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, w.qk[j], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, w.qkl[j], s, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = in_res ? s[i] : s[i] + w.bias;
    s[i] = (t0 + 4 * c + i < n_valid) ? v * a.scale_log2 : -__builtin_inff();
  }

  // ---- V fragments: tokens t0+4c+i, channels n*CPM + j -------------------
  constexpr int VB = CPM * BITS / 8;  // bytes per token of the lane's V slice
  constexpr int VW = VB >= 4 ? VB / 4 : 1;
  uint32_t vw[4][VW];
  const int G = D / L.VG;
  const int g = (n * CPM) / L.VG;
  _Float16 sv[4], mv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tv = t0 + 4 * c + i;
    const long rb = row_base(pages, L, blk, tv, BITS);
    const bool ok = tv < n_valid && rb >= 0;
    if (ok) {
      load_bytes<VB>(pages + rb + side + headb + (long)n * VB, vw[i]);
      const long e = ((long)tv * L.H + h) * G + g;
      sv[i] = *f16p(pages, blk * L.stride + L.o_vs + 2 * e);
      mv[i] = *f16p(pages, blk * L.stride + L.o_vm + 2 * e);
    } else {
#pragma unroll
      for (int k = 0; k < VW; ++k) vw[i][k] = 0;
      sv[i] = (_Float16)0.f;
      mv[i] = (_Float16)0.f;
    }
  }
  const h2_t s01 = {sv[0], sv[1]}, s23 = {sv[2], sv[3]};
  const h2_t m01 = {mv[0], mv[1]}, m23 = {mv[2], mv[3]};
  h4_t va[CPM];
#pragma unroll
  for (int j = 0; j < CPM; ++j) {
    // byte / shift of channel j inside the lane's slice
    constexpr int PER = 8 / BITS;
    const int byte = j / PER, sh = (j % PER) * BITS;
    const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + (byte & 3)) << 16) | (uint32_t)(byte & 3);
    const int wd = byte >> 2;
    const uint32_t mask = ((1u << BITS) - 1u) * 0x00010001u;
    const uint32_t x01 = (__builtin_amdgcn_perm(vw[1][wd], vw[0][wd], sel) >> sh) & mask;
    const uint32_t x23 = (__builtin_amdgcn_perm(vw[3][wd], vw[2][wd], sel) >> sh) & mask;
    const h2_t v01 = __builtin_elementwise_fma(code_pair(x01), s01, m01);
    const h2_t v23 = __builtin_elementwise_fma(code_pair(x23), s23, m23);
    va[j] = h4_t{v01[0], v01[1], v23[0], v23[1]};
  }
  softmax_pv<D, QLO>(w, s, va);
}

// ---------------------------------------------------------------------------
// Tier-specialised pipelined path. Each wave streams its KV head's tiles of the
// split through an NBUF-slot ring in LDS, filled by direct global->LDS DMA
// (global_load_lds_dword{,x4}: lane L's bytes land at slot + size * L), so the
// bytes in flight per CU are set by the ring size, not by VGPRs. The DMAs are
// issued from inline asm: the compiler neither sees them nor inserts waits for
// them; the wave waits with an explicit s_waitcnt vmcnt(n) for the tile it is
// about to read (loads retire in order, so waiting for "at most n outstanding"
// covers every older load). Every tile issues the same number of DMA
// instructions (a tile the fast path does not take -- the open K group, a block
// of another tier -- loads a dummy 16 bytes per lane from its page header), so
// n is a compile-time count.
// ---------------------------------------------------------------------------
#pragma clang diagnostic ignored "-Winline-asm"

__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int D, int BITS>
struct Ring {
  static constexpr int KB = D * BITS / 8;                 // code bytes per token, one side, one head
  static constexpr int KCB = 16 * KB;                     // per tile
  static constexpr int KI = (KCB / 16 + 63) / 64;         // dwordx4 DMAs per side
  static constexpr int OFF_V = KCB, OFF_S = 2 * KCB;      // K codes | V codes | k_scale, k_min | V stats
  static constexpr int OFF_VS = 2 * KCB + 4 * D;
  static constexpr int SLOT = OFF_VS + 16 * 4 * 4;        // V stats for G <= 4 groups
  static constexpr int NBUF = BITS == 8 ? 3 : 4;
  static constexpr int M = 2 * KI + 2;                    // DMA instructions per tile
  static constexpr int WAVE_BYTES = NBUF * SLOT;
};

// Per-block facts of the split's next <= 64 blocks, one block per lane: chunk
// byte offsets (chunk 0 is the block's own page), tier and residual mapping.
struct BlockLane {
  long cb0, cb1, cb2, cb3;
  int blk;    // -1: not a valid block id
  int tier;
  // kNotFast unless the block is stored at the kernel's tier with every chunk it
  // needs in range; else the K group read from the residual (-1: none), whose
  // tile takes the generic path. Derived from the loads (not a loaded register
  // itself), so the compiler waits for them once, before the tile loop, rather
  // than with a vmcnt(0) -- which would drain the DMA ring -- at a use inside it.
  int fast_rg;
  int rslot, rgrp;
};
constexpr int kNotFast = -0x7fffffff;

__device__ __forceinline__ long mul32(long a, long b) { return (long)((uint64_t)(uint32_t)a * (uint32_t)b); }

template <int BITS>
__device__ __forceinline__ BlockLane load_block(const DecodeArgs& a, long blk) {
  const Lay& L = a.L;
  BlockLane b{0, 0, 0, 0, -1, 2, kNotFast, -1, -1};
  if (blk < 0 || blk >= L.nb) return b;
  const long pg = mul32(blk, L.stride);
  const uint4 hd = *(const uint4*)(a.pages + pg);
  b.blk = (int)blk;
  b.tier = tier_of(hd.x & 0xffu);
  b.cb0 = pg + L.o_data;
  const uint32_t ids[3] = {hd.y, hd.z, hd.w};
  long cbs[3];
  bool ok = true;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const uint32_t id = ids[j];
    const uint32_t page = a.kc_mul ? __umulhi(id, a.kc_mul) : id;
    const uint32_t slot = id - page * (uint32_t)L.KC;
    const bool in = (int)id >= 0 && (long)page < L.nb;
    cbs[j] = in ? mul32(page, L.stride) + L.o_data + mul32(slot, L.cb) : b.cb0;
    if (j < (BITS == 8 ? 3 : (BITS == 4 ? 1 : 0))) ok = ok && in;
  }
  b.cb1 = cbs[0];
  b.cb2 = cbs[1];
  b.cb3 = cbs[2];
  const long rs = a.block_res[blk];
  if (rs >= 0 && rs < a.res.rows) {
    b.rslot = (int)rs;
    b.rgrp = (int)a.res_group[rs];
  }
  b.fast_rg = ok && b.tier == BITS ? (b.rgrp < 0 ? -1 : b.rgrp) : kNotFast;
  return b;
}

__device__ __forceinline__ long readlane64(long v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v >> 32), lane);
  return (long)(((uint64_t)hi << 32) | lo);
}

// DMA one tile (16 tokens from block offset t0) of head h into ring slot `slot`;
// a non-fast tile issues the same number of DMAs, each lane 0 copying 4 header bytes.
template <int D, int BITS>
__device__ __forceinline__ void issue_tile(const DecodeArgs& a, uint32_t slot, bool fast, int t0, int h, int lane,
                                           long cb0, long cb1, long cb2, long cb3) {
  using R = Ring<D, BITS>;
  const Lay& L = a.L;
  const uint8_t* page = a.pages + (cb0 - L.o_data);
  if (!fast) {
#pragma unroll
    for (int i = 0; i < R::M; ++i) {
      if (lane == 0) dma4(page, slot);
    }
    return;
  }
  constexpr int LB = BITS == 8 ? 3 : (BITS == 4 ? 2 : 1);
  const int tpc_shift = a.bs_shift + 1 - LB;  // tokens per chunk = 2 * BS / BITS
  constexpr long ROWB = 2L * D * BITS / 8;     // per head; a row holds all heads
  const long rowb = ROWB * L.H;
  const long side = rowb / 2;
  const long headb = (long)h * R::KB;
  constexpr int QPT = R::KB / 16;
#pragma unroll
  for (int r = 0; r < R::KI; ++r) {
    const int idx = lane + 64 * r;
    const int t = t0 + idx / QPT;
    const int j = t >> tpc_shift;
    long cb = cb0;
    if constexpr (BITS >= 4) cb = j == 1 ? cb1 : cb;
    if constexpr (BITS == 8) cb = j == 2 ? cb2 : (j == 3 ? cb3 : cb);
    const uint8_t* src = a.pages + cb + (long)(t & ((1 << tpc_shift) - 1)) * rowb + headb + 16 * (idx % QPT);
    if (idx < R::KCB / 16) {
      dma16(src, slot + 1024 * r);
      dma16(src + side, slot + R::OFF_V + 1024 * r);
    }
  }
  {  // k_scale / k_min of the tile's K group: D/8 lanes each
    const long e0 = (long)((t0 >> a.kg_shift) * L.H + h) * D * 2;
    const uint8_t* src = lane < D / 8 ? page + L.o_ks + e0 + 16 * lane : page + L.o_km + e0 + 16 * (lane - D / 8);
    if (lane < D / 4) dma16(src, slot + R::OFF_S);
  }
  {  // V scale / min: G halves per token each, moved as G/2 dwords
    const int G = D >> a.vg_shift;
    const int sp = G == 4 ? 1 : 0;  // log2(dwords per token per stat)
    const int which = lane >> (4 + sp);
    const int r = lane & ((16 << sp) - 1);
    const int t = t0 + (r >> sp);
    const uint8_t* src = page + (which ? L.o_vm : L.o_vs) + (long)(t * L.H + h) * G * 2 + 4 * (r & ((1 << sp) - 1));
    if (lane < (32 << sp)) dma4(src, slot + R::OFF_VS);
  }
}

// One fast tile from LDS slot `sp` (tier BITS, K from codes).
template <int D, bool QLO, int BITS>
__device__ __forceinline__ void compute_tile(Wave<D, QLO>& w, const DecodeArgs& a, const uint8_t* sp, int t0,
                                             int n_valid, bool new_group, int lane) {
  using W = Wave<D, QLO>;
  using R = Ring<D, BITS>;
  constexpr int CPL = W::CPL, NQK = W::NQK, CPM = W::CPM;
  const int c = lane >> 4, n = lane & 15;
  if (new_group)
    build_qk_at<D, QLO, BITS>(w, sp + R::OFF_S + 2 * c * CPL, sp + R::OFF_S + 2 * D + 2 * c * CPL, n < a.gqa);
  f4_t s = {0.f, 0.f, 0.f, 0.f};
  {
    constexpr int KW = CPL * BITS / 32 > 0 ? CPL * BITS / 32 : 1;
    uint32_t kw[KW];
    load_bytes<CPL * BITS / 8>(sp + n * R::KB + c * (CPL * BITS / 8), kw);
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      uint32_t wj[2];
      if constexpr (BITS == 8) {
        wj[0] = kw[2 * j];
        wj[1] = kw[2 * j + 1];
      } else if constexpr (BITS == 4) {
        wj[0] = kw[j];
      } else {
        wj[0] = kw[j >> 1] >> (16 * (j & 1));
      }
      const h8_t kf = unpack8<BITS>(wj);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, w.qk[j], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, w.qkl[j], s, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = (t0 + 4 * c + i < n_valid) ? (s[i] + w.bias) * a.scale_log2 : -__builtin_inff();

  constexpr int VB = CPM * BITS / 8;
  constexpr int VW = VB >= 4 ? VB / 4 : 1;
  uint32_t vw[4][VW];
  const int G = D >> a.vg_shift;
  const int g = (n * CPM) >> a.vg_shift;
  const _Float16* vs = (const _Float16*)(sp + R::OFF_VS);
  _Float16 sv[4], mv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tv = 4 * c + i;
    load_bytes<VB>(sp + R::OFF_V + tv * R::KB + n * VB, vw[i]);
    const bool ok = t0 + tv < n_valid;
    sv[i] = ok ? vs[tv * G + g] : (_Float16)0.f;
    mv[i] = ok ? vs[16 * G + tv * G + g] : (_Float16)0.f;
  }
  const h2_t s01 = {sv[0], sv[1]}, s23 = {sv[2], sv[3]};
  const h2_t m01 = {mv[0], mv[1]}, m23 = {mv[2], mv[3]};
  h4_t va[CPM];
#pragma unroll
  for (int j = 0; j < CPM; ++j) {
    constexpr int PER = 8 / BITS;
    const int byte = j / PER, sh = (j % PER) * BITS;
    const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + (byte & 3)) << 16) | (uint32_t)(byte & 3);
    const int wd = byte >> 2;
    const uint32_t mask = ((1u << BITS) - 1u) * 0x00010001u;
    const uint32_t x01 = (__builtin_amdgcn_perm(vw[1][wd], vw[0][wd], sel) >> sh) & mask;
    const uint32_t x23 = (__builtin_amdgcn_perm(vw[3][wd], vw[2][wd], sel) >> sh) & mask;
    const h2_t v01 = __builtin_elementwise_fma(code_pair(x01), s01, m01);
    const h2_t v23 = __builtin_elementwise_fma(code_pair(x23), s23, m23);
    va[j] = h4_t{v01[0], v01[1], v23[0], v23[1]};
  }
  softmax_pv<D, QLO>(w, s, va);
}

template <int D, int BITS, int NB>
__device__ __forceinline__ void wait_tile(int ahead) {
  // `ahead` tiles were issued after the one about to be read.
  constexpr int M = Ring<D, BITS>::M;
  if (NB >= 4 && ahead >= 3) wait_vmcnt<3 * M>();
  else if (ahead >= 2) wait_vmcnt<2 * M>();
  else if (ahead == 1) wait_vmcnt<M>();
  else wait_vmcnt<0>();
}

template <int D, int BITS, bool QLO>
__global__ __launch_bounds__(512) void decode_kernel(DecodeArgs a) {
  using W = Wave<D, QLO>;
  using R = Ring<D, BITS>;
  extern __shared__ __attribute__((aligned(16))) uint8_t ring_lds[];
  const Lay& L = a.L;
  const int split = blockIdx.x;
  const long seq = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int h = blockIdx.z * (blockDim.x >> 6) + wv;
  if (h >= L.H) return;
  const int seq_len = (int)a.lens[seq];
  if (seq_len <= 0) return;
  const int n_blocks = (seq_len + L.BS - 1) / L.BS;
  const int per = (n_blocks + a.num_splits - 1) / a.num_splits;
  const int bps = a.bps > per ? a.bps : per;
  const int b_start = split * bps;
  if (b_start >= n_blocks) return;
  const int b_end = b_start + bps < n_blocks ? b_start + bps : n_blocks;
  const long q_row = a.q_rows ? a.q_rows[seq] : seq;
  const long bt_row = a.bt_rows ? a.bt_rows[seq] : seq;
  const int c = lane >> 4, n = lane & 15;
  uint8_t* my_ring = ring_lds + wv * R::WAVE_BYTES;
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)my_ring);

  W w;
  {
    const bool qv = n < a.gqa;
    const long qb = q_row * a.q_s0 + (long)(h * a.gqa + (qv ? n : 0)) * a.q_s1 + c * W::CPL;
    float xq[W::CPL];
    if (qv) {
      ld_n<W::CPL>(a.q, a.q_dtype, qb, xq);
    } else {
#pragma unroll
      for (int e = 0; e < W::CPL; ++e) xq[e] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < W::CPL / 2; ++i) {
      const float x0 = xq[2 * i], x1 = xq[2 * i + 1];
      const h2_t hi = {(_Float16)x0, (_Float16)x1};
      w.qn[i] = h2u(hi);
      if constexpr (QLO) {
        const h2_t lo = {(_Float16)(x0 - (float)hi[0]), (_Float16)(x1 - (float)hi[1])};
        w.ql[i] = h2u(lo);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < W::CPM; ++j) w.acc[j] = f4_t{0.f, 0.f, 0.f, 0.f};
  w.m_run = -__builtin_inff();
  w.l_lane = 0.f;
  w.bias = 0.f;

  const int tpb_shift = a.bs_shift - 4;  // tiles per block = BS / 16
  const bool stats_ok = (D >> a.vg_shift) == 2 || (D >> a.vg_shift) == 4;
  for (int c0 = b_start; c0 < b_end; c0 += 64) {
    const int nb = b_end - c0 < 64 ? b_end - c0 : 64;
    const BlockLane bl = load_block<BITS>(a, lane < nb ? (long)a.bt[bt_row * a.bt_s0 + c0 + lane] : -1L);
    const int last_tok = (c0 + nb) * L.BS < seq_len ? (c0 + nb) * L.BS : seq_len;
    const int n_tiles = (last_tok - c0 * L.BS + 15) >> 4;

    auto issue = [&](int tt) {
      const int b = tt >> tpb_shift;
      const int t0 = (tt & ((1 << tpb_shift) - 1)) << 4;
      const int frg = __builtin_amdgcn_readlane(bl.fast_rg, b);
      const bool fast = frg != kNotFast && frg != (t0 >> a.kg_shift) && stats_ok;
      const long cb0 = readlane64(bl.cb0, b);
      const long cb1 = BITS >= 4 ? readlane64(bl.cb1, b) : cb0;
      const long cb2 = BITS == 8 ? readlane64(bl.cb2, b) : cb0;
      const long cb3 = BITS == 8 ? readlane64(bl.cb3, b) : cb0;
      const uint32_t slot = ring0 + (uint32_t)((tt % R::NBUF) * R::SLOT);
      issue_tile<D, BITS>(a, slot, fast, t0, h, lane, cb0, cb1, cb2, cb3);
    };

#pragma unroll 1
    for (int tt = 0; tt < R::NBUF - 1 && tt < n_tiles; ++tt) issue(tt);
    long qk_blk = -1;
    int qk_grp = -1, qk_bits = 0;
#pragma unroll 1
    for (int tt = 0; tt < n_tiles; ++tt) {
      if (tt + R::NBUF - 1 < n_tiles) issue(tt + R::NBUF - 1);
      const int ahead = (n_tiles - 1 - tt) < (R::NBUF - 1) ? (n_tiles - 1 - tt) : (R::NBUF - 1);
      const int b = tt >> tpb_shift;
      const int t0 = (tt & ((1 << tpb_shift) - 1)) << 4;
      const long blk = __builtin_amdgcn_readlane(bl.blk, b);
      if (blk < 0) continue;
      const int grp = t0 >> a.kg_shift;
      const int frg = __builtin_amdgcn_readlane(bl.fast_rg, b);
      const bool fast = frg != kNotFast && frg != grp && stats_ok;
      const int n_valid = seq_len - ((c0 + b) << a.bs_shift);
      if (fast) {
        wait_tile<D, BITS, R::NBUF>(ahead);
        const bool new_group = blk != qk_blk || grp != qk_grp || qk_bits != BITS;
        compute_tile<D, QLO, BITS>(w, a, my_ring + (tt % R::NBUF) * R::SLOT, t0, n_valid, new_group, lane);
        qk_blk = blk;
        qk_grp = grp;
        qk_bits = BITS;
      } else {
        const int tier = __builtin_amdgcn_readlane(bl.tier, b);
        const int rgrp = __builtin_amdgcn_readlane(bl.rgrp, b);
        const long rslot = __builtin_amdgcn_readlane(bl.rslot, b);
        const bool in_res = rslot >= 0 && rgrp == grp;
        if (!in_res && (blk != qk_blk || grp != qk_grp || tier != qk_bits)) {
          if (tier == 4) build_qk<D, QLO, 4>(w, a.pages, L, blk, grp, h, c, n < a.gqa);
          else if (tier == 8) build_qk<D, QLO, 8>(w, a.pages, L, blk, grp, h, c, n < a.gqa);
          else build_qk<D, QLO, 2>(w, a.pages, L, blk, grp, h, c, n < a.gqa);
          qk_blk = blk;
          qk_grp = grp;
          qk_bits = tier;
        }
        if (tier == 4) tile<D, QLO, 4>(w, a, blk, t0, n_valid, rslot, in_res, h, lane);
        else if (tier == 8) tile<D, QLO, 8>(w, a, blk, t0, n_valid, rslot, in_res, h, lane);
        else tile<D, QLO, 2>(w, a, blk, t0, n_valid, rslot, in_res, h, lane);
      }
    }
    wait_vmcnt<0>();  // nothing of this chunk may still be landing in the ring
  }

  float l = w.l_lane;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (n < a.gqa) {
    const long qh = (long)h * a.gqa + n;
    const long row = (seq * a.hq + qh) * a.num_splits + split;
    float* dst = a.acc + row * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < W::CPM; ++j) dst[(4 * c + i) * W::CPM + j] = w.acc[j][i];
    }
    if (c == 0) {
      a.ml[row * 2] = w.m_run;
      a.ml[row * 2 + 1] = l;
    }
  }
}

__global__ __launch_bounds__(64) void merge_kernel(MergeArgs a) {
  const long seq = blockIdx.x;
  const int head = blockIdx.y;
  const int seq_len = (int)a.lens[seq];
  if (seq_len <= 0) return;
  const int n_blocks = (seq_len + a.BS - 1) / a.BS;
  const int per = (n_blocks + a.num_splits - 1) / a.num_splits;
  const int bps = a.bps > per ? a.bps : per;
  const int used = (n_blocks + bps - 1) / bps;
  const long base = (seq * a.hq + head) * a.num_splits;
  float m = -__builtin_inff();
  for (int sp = 0; sp < used; ++sp) m = fmaxf(m, a.ml[(base + sp) * 2]);
  const long o_row = a.q_rows ? a.q_rows[seq] : seq;
  for (int d = threadIdx.x; d < a.D; d += 64) {
    float num = 0.f, den = 0.f;
    for (int sp = 0; sp < used; ++sp) {
      const float wgt = __builtin_amdgcn_exp2f(a.ml[(base + sp) * 2] - m);
      den += a.ml[(base + sp) * 2 + 1] * wgt;
      num += a.acc[(base + sp) * a.D + d] * wgt;
    }
    st(a.out, a.out_dtype, o_row * a.o_s0 + head * a.o_s1 + d, num / den);
  }
}

template <int D, int BITS, bool QLO>
hipError_t launch_decode_t(const DecodeArgs& a, dim3 grid, dim3 block, hipStream_t s) {
  const size_t lds = (size_t)(block.x / 64) * Ring<D, BITS>::WAVE_BYTES;
  static bool attr = false;  // idempotent; set once per instantiation
  if (!attr) {
    if (hipFuncSetAttribute((const void*)decode_kernel<D, BITS, QLO>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return hipErrorInvalidValue;
    attr = true;
  }
  hipLaunchKernelGGL((decode_kernel<D, BITS, QLO>), grid, block, lds, s, a);
  return hipGetLastError();
}

template <int D, bool QLO>
hipError_t launch_decode_d(const DecodeArgs& a, dim3 grid, dim3 block, hipStream_t s) {
  if (a.tier == 8) return launch_decode_t<D, 8, QLO>(a, grid, block, s);
  if (a.tier == 2) return launch_decode_t<D, 2, QLO>(a, grid, block, s);
  return launch_decode_t<D, 4, QLO>(a, grid, block, s);
}

hipError_t launch_decode(const DecodeArgs& a, long num_seqs, hipStream_t s) {
  const int hpw = a.L.H < 8 ? a.L.H : 8;
  const dim3 grid((unsigned)a.num_splits, (unsigned)num_seqs, (unsigned)((a.L.H + hpw - 1) / hpw));
  const dim3 block(64 * hpw);
  const bool qlo = a.q_dtype == ECHOKV_F32;
  if (a.L.D == 128) return qlo ? launch_decode_d<128, true>(a, grid, block, s) : launch_decode_d<128, false>(a, grid, block, s);
  if (a.L.D == 64) return qlo ? launch_decode_d<64, true>(a, grid, block, s) : launch_decode_d<64, false>(a, grid, block, s);
  return hipErrorInvalidValue;
}

hipError_t launch_merge(const MergeArgs& a, long num_seqs, hipStream_t s) {
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)num_seqs, (unsigned)a.hq), dim3(64), 0, s, a);
  return hipGetLastError();
}

}  // namespace ek
