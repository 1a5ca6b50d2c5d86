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

template <int D, bool QLO, int BITS>
__device__ __forceinline__ void build_qk(Wave<D, QLO>& w, const uint8_t* pages, const Lay& L, long blk, int grp,
                                         int h, int c) {
  constexpr int CPL = Wave<D, QLO>::CPL;
  const long e0 = ((long)grp * L.H + h) * D + c * CPL;
  uint32_t ks[CPL / 2], km[CPL / 2];
  load_bytes<2 * CPL>(pages + blk * L.stride + L.o_ks + 2 * e0, ks);
  load_bytes<2 * CPL>(pages + blk * L.stride + L.o_km + 2 * e0, km);
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
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      h8_t kh, kl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = kvalid ? ld(a.res.ptr, a.res.dtype, r0 + 8 * j + e) : 0.f;
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

template <int D, bool QLO>
__global__ __launch_bounds__(512) void decode_kernel(DecodeArgs a) {
  using W = Wave<D, QLO>;
  const Lay& L = a.L;
  const int split = blockIdx.x;
  const long seq = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.z * (blockDim.x >> 6) + (threadIdx.x >> 6);
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

  W w;
  {
    const bool qv = n < a.gqa;
    const long qb = q_row * a.q_s0 + (long)(h * a.gqa + (qv ? n : 0)) * a.q_s1 + c * W::CPL;
#pragma unroll
    for (int i = 0; i < W::CPL / 2; ++i) {
      const float x0 = qv ? ld(a.q, a.q_dtype, qb + 2 * i) : 0.f;
      const float x1 = qv ? ld(a.q, a.q_dtype, qb + 2 * i + 1) : 0.f;
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

  long qk_blk = -1;
  int qk_grp = -1, qk_bits = 0;
  for (int bi = b_start; bi < b_end; ++bi) {
    const long blk = a.bt[bt_row * a.bt_s0 + bi];
    if (blk < 0 || blk >= L.nb) continue;
    const int bits = tier_of(a.pages[blk * L.stride]);
    const long rslot = a.block_res[blk];
    const long rgrp = (rslot >= 0 && rslot < a.res.rows) ? a.res_group[rslot] : -1;
    const int n_valid = seq_len - bi * L.BS;
    for (int t0 = 0; t0 < L.BS && t0 < n_valid; t0 += 16) {
      const int grp = t0 / L.KG;
      const bool in_res = rgrp == grp;
      if (!in_res && (blk != qk_blk || grp != qk_grp || bits != qk_bits)) {
        if (bits == 4) build_qk<D, QLO, 4>(w, a.pages, L, blk, grp, h, c);
        else if (bits == 8) build_qk<D, QLO, 8>(w, a.pages, L, blk, grp, h, c);
        else build_qk<D, QLO, 2>(w, a.pages, L, blk, grp, h, c);
        qk_blk = blk;
        qk_grp = grp;
        qk_bits = bits;
      }
      if (bits == 4) tile<D, QLO, 4>(w, a, blk, t0, n_valid, rslot, in_res, h, lane);
      else if (bits == 8) tile<D, QLO, 8>(w, a, blk, t0, n_valid, rslot, in_res, h, lane);
      else tile<D, QLO, 2>(w, a, blk, t0, n_valid, rslot, in_res, h, lane);
    }
  }

  // Row sums live per lane (4 tokens each); reduce across the 4 lane groups.
  float l = w.l_lane;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (n < a.gqa) {
    const long qh = (long)h * a.gqa + n;
    const long row = (seq * a.hq + qh) * a.num_splits + split;
    float* dst = a.acc + row * D;
    // lane holds channels (4c + i) * CPM + j
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

hipError_t launch_decode(const DecodeArgs& a, long num_seqs, hipStream_t s) {
  const int hpw = a.L.H < 8 ? a.L.H : 8;
  const dim3 grid((unsigned)a.num_splits, (unsigned)num_seqs, (unsigned)((a.L.H + hpw - 1) / hpw));
  const dim3 block(64 * hpw);
  const bool qlo = a.q_dtype == ECHOKV_F32;
  if (a.L.D == 128) {
    if (qlo) hipLaunchKernelGGL((decode_kernel<128, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((decode_kernel<128, false>), grid, block, 0, s, a);
  } else if (a.L.D == 64) {
    if (qlo) hipLaunchKernelGGL((decode_kernel<64, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((decode_kernel<64, false>), grid, block, 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_merge(const MergeArgs& a, long num_seqs, hipStream_t s) {
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)num_seqs, (unsigned)a.hq), dim3(64), 0, s, a);
  return hipGetLastError();
}

}  // namespace ek
