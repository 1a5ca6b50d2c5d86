// Split-KV paged decode attention over the tiered (INT2/INT4/INT8) pages, gfx950.
//
// Work decomposition: a work item is (sequence, split, group of <= 4 KV heads),
// one 64-wide wave per KV head, one workgroup per non-empty item. The heads of
// a token row sit side by side in a page ([K codes of all heads | V codes of
// all heads]), so the waves of a workgroup read neighbouring slices of the same
// cache lines together.
//
// Per 16-token tile a wave runs two MFMA contractions with no transposes:
//   S^T[t, q]  = sum_d codes[t, d] * (q[q, d] * k_scale[d]) + sum_d q[q, d] * k_min[d]
//                (v_mfma_f32_16x16x32_f16; the K scale is folded into the query,
//                 the K min term is one more contraction of k_min with q into
//                 the same accumulator; the block's open K group reads the
//                 full-precision residual instead)
//   O^T[d, q] += V[t, d]^T * P^T[t, q]   (v_mfma_f32_16x16x32_f16, with V = codes *
//                 (scale hi + scale lo) + min and P = p hi + p lo, every part an
//                 exact fp16 operand: the scale split so that codes * part fits
//                 fp16's 11 bits; K = 32 holds the lane's 4 tokens twice, so one
//                 MFMA takes both scale parts against p hi, one more against p lo;
//                 the min, the same for the lane's channels, in one more MFMA)
// Codes are exact in fp16. The query-side operand (q * k_scale, and the residual
// keys) is carried as an fp16 hi + lo pair -- lo = fma(q, s, -hi) rounded once --
// contracted into one fp32 accumulator, so S is accurate to ~2^-22 instead of
// fp16's 2^-11: keys with large outlier channels would otherwise dominate the
// error. Likewise V and P: a value of an outlier channel (|v| ~ 40) rounded to
// fp16 is off by up to 2^-6, and weights rounded to fp16 (2^-12 each) move an
// output whose values spread over +-40 by ~2e-3.
// Lane (c, n) = (lane / 16, lane % 16) of the S^T product holds token n and
// channels [c * D/4, (c+1) * D/4) in natural order; the S^T accumulator layout
// (lane = 4 tokens x 1 query column) is what the second MFMA's B operand takes
// (the lane's 4 tokens, twice over K = 32), and the O^T accumulator keeps one
// query column per lane, so the online softmax runs per lane with two cross-row
// max reductions per tile (v_permlane16_swap / v_permlane32_swap). Query
// columns are the GQA heads of the KV head, padded to 16. Codes become fp16
// exactly: INT8 bytes under the exponent of 1024 (0x6400) -- V then subtracts
// 1024, K keeps 1024 + c and removes 1024 * sum(q * k_scale) with one more MFMA
// contraction -- and INT2 / INT4 through gfx950's fp8 conversion (a byte b < 16
// read as E4M3 and scaled by 2^9 is b itself); v_perm_b32 gathers the code bytes.
// The running max is rescaled lazily: only when some column's max grows by more
// than 2^8 (probabilities stay <= 256, far inside fp16).
//
// A split covers max(blocks_per_split, ceil(blocks / num_splits)) blocks of
// the sequence's own length, so results do not depend on the rest of the
// batch; a second kernel merges the splits in order (log-sum-exp, log2 units).
#include "args.h"

namespace ek {

typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h2_t u2h(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t h2u(h2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ h8_t w2h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(h8_t, u4_t{a, b, c, d});
}

constexpr float kLazyRescale = 8.0f;  // log2 units
// KV heads (waves) per workgroup: 4 lets two or three workgroups share a CU, so
// one's start-up (query, block table and header loads) overlaps another's tiles.
constexpr int kHeadsPerGroup = 4;

// v_perm_b32 selector: byte `a` of the low source to bits 0-7, byte `b` of the
// high source to bits 16-23, zeros elsewhere (perm(hi, lo, sel)).
constexpr uint32_t pair_sel(int a, int b) { return 0x0C000C00u | ((uint32_t)(4 + b) << 16) | (uint32_t)a; }
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Code unpacking constants, held in registers: GFX9 VOP3 instructions take no
// literal operand, so with both in registers (one of them scalar) the
// mask-and-insert-exponent step is one v_and_or_b32 instead of v_and + v_or.
struct CodeK {
  uint32_t mask;   // the code bits of each 16-bit half (scalar register)
  uint32_t magic;  // 0x64006400: the exponent of 1024 in each half (vector register)
};
template <int BITS>
__device__ __forceinline__ CodeK code_consts() {
  CodeK k{BITS == 4 ? 0x000F000Fu : (BITS == 8 ? 0x00FF00FFu : 0x00030003u), 0x64006400u};
  asm volatile("" : "+s"(k.mask));
  asm volatile("" : "+v"(k.magic));
  return k;
}

// INT4 / INT2 codes as fp16 without a bias: a byte b < 16 read as an OCP E4M3
// fp8 value is exactly b * 2^-9, so gfx950's fp8 -> fp16 conversion with the
// scale 2^9 gives the code itself. Two bytes (0-1, or 2-3 with HI) per call.
template <bool HI>
__device__ __forceinline__ uint32_t cvt_codes(uint32_t bytes) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(bytes, 512.0f, HI));
}

// (x & mask) holds two codes at bits 0.. and 16..; as the fp16 pair 1024 + c (exact).
__device__ __forceinline__ uint32_t biased_pair(uint32_t x, const CodeK& k) { return (x & k.mask) | k.magic; }
// ... and as c itself.
__device__ __forceinline__ h2_t code_pair(uint32_t x, const CodeK& k) {
  const h2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  return u2h(biased_pair(x, k)) - k1024;
}

// Eight consecutive channels of a K row, natural order, as an MFMA fragment.
// INT4: one word (8 nibbles); INT2: bytes 2*hf, 2*hf+1 of one word -- both as
// the codes themselves (cvt_codes); INT8: two words, as 1024 + code (s_block
// takes the bias back out with one more contraction).
template <int BITS>
__device__ __forceinline__ h8_t kfrag(const uint32_t* w, int hf, const CodeK& k) {
  if constexpr (BITS == 4) {
    const uint32_t x = w[0];
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;  // even / odd channels, one per byte
    const uint32_t c03 = perm(hi, lo, 0x05010400u), c47 = perm(hi, lo, 0x07030602u);
    (void)k;
    return w2h8(cvt_codes<false>(c03), cvt_codes<true>(c03), cvt_codes<false>(c47), cvt_codes<true>(c47));
  } else if constexpr (BITS == 8) {
    const uint32_t m = 0x64646464u;  // perm(m, x, ...) puts 0x64 above each code byte
    return w2h8(perm(m, w[0], 0x04010400u), perm(m, w[0], 0x04030402u), perm(m, w[1], 0x04010400u),
                perm(m, w[1], 0x04030402u));
  } else {
    // y_k: code k of every byte (byte b holds channels 4b .. 4b+3); a v_perm
    // puts channels (k, k+1) of byte 2hf next to each other, (4+k, 5+k) of
    // byte 2hf+1 above them.
    const uint32_t x = w[0];
    const uint32_t y0 = x & 0x03030303u, y1 = (x >> 2) & 0x03030303u;
    const uint32_t y2 = (x >> 4) & 0x03030303u, y3 = (x >> 6) & 0x03030303u;
    const uint32_t b0 = 2 * hf, b1 = 2 * hf + 1;
    const uint32_t sel = b0 | ((4 + b0) << 8) | (b1 << 16) | ((4 + b1) << 24);
    const uint32_t p01 = perm(y1, y0, sel), p23 = perm(y3, y2, sel);
    (void)k;
    return w2h8(cvt_codes<false>(p01), cvt_codes<false>(p23), cvt_codes<true>(p01), cvt_codes<true>(p23));
  }
}

// Eight byte-wide codes (two words) as an MFMA fragment of the codes themselves:
// 1024 + c minus 1024 is exact in fp16. Unlike kfrag<8>, no 1024 bias enters the
// fp32 score sums, whose rounding would otherwise scale with 1024 * |q * k_scale|
// rather than with the score (INT2 / INT4 codes are small next to the bias).
__device__ __forceinline__ h8_t kfrag_bytes(const uint32_t* w) {
  const uint32_t m = 0x64646464u;
  const h2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const h2_t a = u2h(perm(m, w[0], 0x04010400u)) - k1024, b = u2h(perm(m, w[0], 0x04030402u)) - k1024;
  const h2_t c = u2h(perm(m, w[1], 0x04010400u)) - k1024, d = u2h(perm(m, w[1], 0x04030402u)) - k1024;
  return w2h8(h2u(a), h2u(b), h2u(c), h2u(d));
}

// Fragment j (channels 8j..8j+7 of the lane's slice) from the lane's K words.
template <int BITS>
__device__ __forceinline__ h8_t kfrag_j(const uint32_t* kw, int j, const CodeK& k) {
  if constexpr (BITS == 4) return kfrag<4>(kw + j, 0, k);
  else if constexpr (BITS == 8) return kfrag<8>(kw + 2 * j, 0, k);
  else return kfrag<2>(kw + (j >> 1), j & 1, k);
}

// The codes of the lane's V channel j for its 4 tokens, as fp16 (exact): v[i] =
// token i's slice words, vs = pre-shifted copies. pv_tile dequantizes them.
template <int BITS, int VW>
__device__ __forceinline__ h4_t vfrag(int j, const uint32_t (*v)[VW], const uint32_t (*vs)[4], const CodeK& k) {
  uint32_t x01, x23;
  if constexpr (BITS == 4) {
    const int by = j >> 1, sh = j & 1;  // odd channels: low nibble of the word >> 4
    x01 = perm(vs[1][sh], vs[0][sh], pair_sel(by, by));
    x23 = perm(vs[3][sh], vs[2][sh], pair_sel(by, by));
  } else if constexpr (BITS == 8) {
    const int wd = j >> 2, by = j & 3;
    x01 = perm(v[1][wd], v[0][wd], pair_sel(by, by));
    x23 = perm(v[3][wd], v[2][wd], pair_sel(by, by));
  } else {
    const int by = j >> 2, sh = j & 3;  // code j at bits 2*sh of byte by
    x01 = perm(vs[1][sh], vs[0][sh], pair_sel(by, by));
    x23 = perm(vs[3][sh], vs[2][sh], pair_sel(by, by));
  }
  const h2_t c01 = code_pair(x01, k), c23 = code_pair(x23, k);
  return h4_t{c01[0], c01[1], c23[0], c23[1]};
}

// INT4 V^T codes of all the lane's CPM (4 or 8) channels: a v_perm pairs the
// bytes of tokens (0, 1) or (2, 3) holding four channels, the nibbles split into
// even / odd channels one per byte, cvt_codes makes the exact fp16 codes.
template <int CPM>
__device__ __forceinline__ void vfrags4(const uint32_t (*v)[1], h4_t* va) {
  static_assert(CPM == 4 || CPM == 8, "INT4 V: the lane's channels of a token fit one word");
#pragma unroll
  for (int hb = 0; hb < CPM / 4; ++hb) {  // bytes 2hb, 2hb+1 of each token: channels 4hb .. 4hb+3
    const uint32_t sel = (uint32_t)(2 * hb) | ((uint32_t)(4 + 2 * hb) << 8) | ((uint32_t)(2 * hb + 1) << 16) |
                         ((uint32_t)(4 + 2 * hb + 1) << 24);
    const uint32_t x01 = perm(v[1][0], v[0][0], sel), x23 = perm(v[3][0], v[2][0], sel);
    const uint32_t e01 = x01 & 0x0F0F0F0Fu, o01 = (x01 >> 4) & 0x0F0F0F0Fu;  // even / odd channels
    const uint32_t e23 = x23 & 0x0F0F0F0Fu, o23 = (x23 >> 4) & 0x0F0F0F0Fu;
    auto frag = [&](uint32_t c01, uint32_t c23) {
      const h2_t a0 = u2h(c01), a1 = u2h(c23);
      return h4_t{a0[0], a0[1], a1[0], a1[1]};
    };
    va[4 * hb] = frag(cvt_codes<false>(e01), cvt_codes<false>(e23));
    va[4 * hb + 1] = frag(cvt_codes<false>(o01), cvt_codes<false>(o23));
    va[4 * hb + 2] = frag(cvt_codes<true>(e01), cvt_codes<true>(e23));
    va[4 * hb + 3] = frag(cvt_codes<true>(o01), cvt_codes<true>(o23));
  }
}

// INT2 V^T codes of the lane's CPM (4 or 8) channels: a v_perm interleaves
// the code bytes of tokens (0, 1) / (2, 3) (byte b holds channels 4b .. 4b+3),
// so each shift-and-mask leaves channel k of both tokens in bytes 0-1 and
// channel 4+k in bytes 2-3, as cvt_codes takes them.
template <int CPM>
__device__ __forceinline__ void vfrags2(const uint32_t (*v)[1], h4_t* va) {
  static_assert(CPM == 4 || CPM == 8, "INT2 V: the lane's channels of a token fit one word");
  const uint32_t sel = 0x05010400u;  // t0.b0, t1.b0, t0.b1, t1.b1
  const uint32_t x01 = perm(v[1][0], v[0][0], sel), x23 = perm(v[3][0], v[2][0], sel);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t c01 = (x01 >> (2 * k)) & 0x03030303u, c23 = (x23 >> (2 * k)) & 0x03030303u;
    auto frag = [&](uint32_t a01, uint32_t a23) {
      const h2_t a0 = u2h(a01), a1 = u2h(a23);
      return h4_t{a0[0], a0[1], a1[0], a1[1]};
    };
    va[k] = frag(cvt_codes<false>(c01), cvt_codes<false>(c23));
    if constexpr (CPM == 8) va[4 + k] = frag(cvt_codes<true>(c01), cvt_codes<true>(c23));
  }
}

// Shifted copies of the V words that vfrag reads (INT4: >> 0, 4; INT2: >> 0, 2, 4, 6).
template <int BITS, int VW>
__device__ __forceinline__ void vshift(const uint32_t (*v)[VW], uint32_t (*vs)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    vs[i][0] = v[i][0];
    if constexpr (BITS == 4) vs[i][1] = v[i][0] >> 4;
    if constexpr (BITS == 2) {
      vs[i][1] = v[i][0] >> 2;
      vs[i][2] = v[i][0] >> 4;
      vs[i][3] = v[i][0] >> 6;
    }
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

// max without the NaN-quieting canonicalizations fmaxf adds around values of
// unknown origin (the scores are never NaN: masked ones are -inf). Never give
// these an MFMA result directly: the compiler places the wait states an MFMA's
// result needs before its first VALU reader only for instructions it can see,
// so an asm reader could see the accumulator before the MFMA has written it.
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Cross-row (lanes l, l^16, l^32, l^48) reductions; every lane gets the result.
__device__ __forceinline__ float rows_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Per-wave decode state for head_dim D. QLO: the query has a low part (float32 input).
template <int D, bool QLO>
struct Wave {
  static constexpr int CPL = D / 4;   // K channels per lane in the QK fragments
  static constexpr int NQK = D / 32;  // 16x16x32 MFMAs per tile for S^T (per hi / lo chain)
  static constexpr int CPM = D / 16;  // V channels per lane = 16x16x16 MFMAs per tile
  uint32_t qn[CPL / 2];               // fp16 query pairs (hi), natural channel order
  uint32_t ql[QLO ? CPL / 2 : 1];     // fp16 query pairs (lo = q - hi)
  f4_t acc[CPM];                      // O^T fragments: sum_t p * codes * V scale
  f4_t acc_m;                         // sum_t p * V min of the lane's V group (every channel of it)
  float acc_ml;                       // PS: this lane's tokens' share of sum_t w * V min of its column's group
  float m_run, l_lane;                // running max (scaled log2 units), this lane's sum
  float scale;                        // |softmax scale| * log2(e), > 0 (a negative scale negates the query)
};

// S^T of one 16-token tile from its codes, K group by 32-channel block j:
//   S^T += codes_j . (q * k_scale)_j^T   as fp16 hi / lo pairs (one fp32 accumulator:
//                                         lo terms are ~2^-11 of hi, far above its rounding)
//        - 1024 * sum_d (q * k_scale)_j  (BITS 8: fragments carry 1024 + c;
//                                           any other BITS: the codes themselves)
//        + k_min_j . q_j^T               (and q lo for float32 queries)
// The products q * s are exact in fp32; hi = fp16(q * s), lo = fp16(fma(q, s,
// -hi)) keeps S accurate to ~2^-22 relative. Each block's operands are built
// right before its MFMAs, so only one block's live at a time. ks / km: the
// lane's k_scale / k_min words of block j (channels 8 at a time, natural order).
template <int D, bool QLO, int BITS>
__device__ __forceinline__ void s_block(const Wave<D, QLO>& w, const uint32_t* ks, const uint32_t* km,
                                        const h8_t& kf, int j, f4_t& s) {
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h2_t q = u2h(w.qn[4 * j + i]), sc = u2h(ks[i]);
    const h2_t ph = q * sc;
    h2_t pl = __builtin_elementwise_fma(q, sc, -ph);  // exact product minus its rounding, rounded once
    if constexpr (QLO) pl = __builtin_elementwise_fma(u2h(w.ql[4 * j + i]), sc, pl);
    hi[i] = h2u(ph);
    lo[i] = h2u(pl);
  }
  const h8_t h8 = w2h8(hi[0], hi[1], hi[2], hi[3]), l8 = w2h8(lo[0], lo[1], lo[2], lo[3]);
  const h8_t m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f, (_Float16)-1024.0f, (_Float16)-1024.0f,
                      (_Float16)-1024.0f, (_Float16)-1024.0f, (_Float16)-1024.0f, (_Float16)-1024.0f};
  const h8_t mn = w2h8(km[0], km[1], km[2], km[3]);
  s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, h8, s, 0, 0, 0);
  s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, l8, s, 0, 0, 0);
  if constexpr (BITS == 8) {  // INT4 / INT2 fragments carry the codes themselves
    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(m1024, h8, s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(m1024, l8, s, 0, 0, 0);
  } else {
    (void)m1024;
  }
  s = __builtin_amdgcn_mfma_f32_16x16x32_f16(
      mn, w2h8(w.qn[4 * j], w.qn[4 * j + 1], w.qn[4 * j + 2], w.qn[4 * j + 3]), s, 0, 0, 0);
  if constexpr (QLO)
    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(
        mn, w2h8(w.ql[4 * j], w.ql[4 * j + 1], w.ql[4 * j + 2], w.ql[4 * j + 3]), s, 0, 0, 0);
}

// S^T of a tile whose keys are the block's open K group, read from the
// full-precision residual (row = token % KG) and split into fp16 hi + lo
// (fp16 / bf16 keys are exact in fp16: lo = 0 is skipped). Lane (c, n): token
// t0 + n, channels [c * D/4, (c+1) * D/4), eight at a time, of the head whose
// channels start rh elements into a residual row. The residual's dtype is a
// template parameter, so every row load issues before the first MFMA waits.
template <int D, bool QLO, int RDT>
__device__ __forceinline__ void s_from_residual(const Wave<D, QLO>& w, const DecodeArgs& a, long rslot, int t0,
                                                long rh, int lane, f4_t& s) {
  constexpr int CPL = D / 4, NJ = D / 32;
  // Rows loaded together: f32 rows take twice the registers, and hi + lo halves.
  constexpr int STEP = RDT == ECHOKV_F32 ? 2 : NJ;
  const int c = lane >> 4, n = lane & 15;
  const long r0 = rslot * a.res.s0 + (long)((t0 + n) & (a.L.KG - 1)) * a.res.s1 + rh + c * CPL;
#pragma unroll
  for (int j0 = 0; j0 < NJ; j0 += STEP) {
    h8_t kh[STEP], kl[STEP];
#pragma unroll
    for (int u = 0; u < STEP; ++u) {
      const long e0 = r0 + 8 * (j0 + u);
      if constexpr (RDT == ECHOKV_F16) {
        const _Float16* src = (const _Float16*)a.res.ptr + e0;
#pragma unroll
        for (int e = 0; e < 8; ++e) kh[u][e] = src[e];
      } else if constexpr (RDT == ECHOKV_BF16) {
        const uint16_t* src = (const uint16_t*)a.res.ptr + e0;
#pragma unroll
        for (int e = 0; e < 8; ++e) kh[u][e] = (_Float16)bf16_to_f32(src[e]);
      } else {
        const float* src = (const float*)a.res.ptr + e0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = src[e];
          kh[u][e] = (_Float16)v;
          kl[u][e] = (_Float16)(v - (float)kh[u][e]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < STEP; ++u) {
      const int j = j0 + u;
      const h8_t qh = w2h8(w.qn[4 * j], w.qn[4 * j + 1], w.qn[4 * j + 2], w.qn[4 * j + 3]);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[u], qh, s, 0, 0, 0);
      if constexpr (RDT == ECHOKV_F32) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl[u], qh, s, 0, 0, 0);
      if constexpr (QLO) {
        const h8_t ql = w2h8(w.ql[4 * j], w.ql[4 * j + 1], w.ql[4 * j + 2], w.ql[4 * j + 3]);
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[u], ql, s, 0, 0, 0);
      }
    }
  }
}

// The V statistics of the lane's 4 tokens (tokens past the sequence: 0) and the
// split of their scales that makes every PV operand exact in fp16: s = hi + lo,
// hi keeping the leading 11 - BITS significant bits, so codes * hi fits fp16's
// 11 bits exactly, and so does codes * lo for 2- and 4-bit codes (8-bit: lo is
// under a quarter of s, its product rounded to ~2^-14 of codes * s).
struct VStats {
  h2_t s01, s23, m01, m23;
};
template <int BITS>
constexpr uint32_t vscale_mask() {
  return BITS == 8 ? 0xFF00FF00u : (BITS == 4 ? 0xFFF0FFF0u : 0xFFFCFFFCu);
}

// The lane's V codes of its 4 tokens, still packed as loaded (VW words a token),
// and their statistics. The codes become fp16 only after the softmax, so only
// the packed words stay live across it.
template <int VW>
struct VTile {
  uint32_t w[4][VW];
  VStats st;
};

template <int BITS, int CPM, int VW>
__device__ __forceinline__ void v_codes(const uint32_t (*vw)[VW], h4_t* va) {
  if constexpr (BITS == 4) {
    vfrags4<CPM>(vw, va);
  } else if constexpr (BITS == 2) {
    vfrags2<CPM>(vw, va);
  } else {
    uint32_t vsh[4][4];
    vshift<BITS, VW>(vw, vsh);
    const CodeK vk = code_consts<BITS>();
#pragma unroll
    for (int j = 0; j < CPM; ++j) va[j] = vfrag<BITS, VW>(j, vw, vsh, vk);
  }
}

// The lane's V codes of channels j in [P * CPM / 2, (P + 1) * CPM / 2) (half of its
// channels), as v_codes: va[j - P * CPM / 2].
template <int BITS, int CPM, int VW, int P>
__device__ __forceinline__ void v_codes_half(const uint32_t (*vw)[VW], h4_t* va) {
  h4_t all[CPM];
  v_codes<BITS, CPM, VW>(vw, all);  // the other half's conversions are dead code
#pragma unroll
  for (int j = 0; j < CPM / 2; ++j) va[j] = all[P * CPM / 2 + j];
}

// Online-softmax update with the tile's unscaled scores x (masked: -inf), then
// O^T += V^T P^T with V = codes * (s hi + s lo) + min and P = p hi + p lo, and
// the min term in acc_m (the lane's rows share one V group, so its rows of acc_m
// are the min term of every channel it holds). No operand is rounded. p =
// exp2(scale * x - m): the scale rides in the fma.
template <int D, bool QLO, int BITS, int VW>
__device__ __forceinline__ void softmax_pv(Wave<D, QLO>& w, const float* x, const VTile<VW>& vt, uint32_t smask) {
  const VStats& vs = vt.st;
  const float mt = rows_max(vmax(vmax3(x[0], x[1], x[2]), x[3])) * w.scale;
  const float m_new = vmax(w.m_run, mt);
  if (__builtin_amdgcn_ballot_w64(m_new > w.m_run + kLazyRescale)) {
    const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_new);  // m_run = -inf at the start: 0
    w.l_lane *= alpha;
#pragma unroll
    for (int j = 0; j < Wave<D, QLO>::CPM; ++j) w.acc[j] *= alpha;
    w.acc_m *= alpha;
    w.m_run = m_new;
  }
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], w.scale, -w.m_run));
  w.l_lane += (p[0] + p[1]) + (p[2] + p[3]);
  // p = hi + lo in fp16 (lo = the rounding of hi, rounded once: p to ~2^-22).
  const h4_t ph = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
  const h4_t pl = {(_Float16)(p[0] - (float)ph[0]), (_Float16)(p[1] - (float)ph[1]), (_Float16)(p[2] - (float)ph[2]),
                   (_Float16)(p[3] - (float)ph[3])};
  h4_t va[Wave<D, QLO>::CPM];
  v_codes<BITS, Wave<D, QLO>::CPM, VW>(vt.w, va);
  const h2_t sh01 = u2h(h2u(vs.s01) & smask), sh23 = u2h(h2u(vs.s23) & smask);
  const h2_t sl01 = vs.s01 - sh01, sl23 = vs.s23 - sh23;  // exact: the dropped bits
  const h4_t shi = {sh01[0], sh01[1], sh23[0], sh23[1]}, slo = {sl01[0], sl01[1], sl23[0], sl23[1]};
  // 16x16x32 products whose K runs over the lane's 4 tokens twice: element e of
  // a lane's operands is token 4c + (e & 3), A's halves the two scale parts, B's
  // both p hi, then both p lo -- every product of the four parts, each exact.
  const h8_t bh = __builtin_shufflevector(ph, ph, 0, 1, 2, 3, 4, 5, 6, 7);
  const h8_t bl = __builtin_shufflevector(pl, pl, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
  for (int j = 0; j < Wave<D, QLO>::CPM; ++j) {
    const h8_t a = __builtin_shufflevector(va[j] * shi, va[j] * slo, 0, 1, 2, 3, 4, 5, 6, 7);
    w.acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh, w.acc[j], 0, 0, 0);
    w.acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl, w.acc[j], 0, 0, 0);
  }
  const h4_t mins = {vs.m01[0], vs.m01[1], vs.m23[0], vs.m23[1]};
  w.acc_m = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_shufflevector(mins, mins, 0, 1, 2, 3, 4, 5, 6, 7),
                                                   __builtin_shufflevector(ph, pl, 0, 1, 2, 3, 4, 5, 6, 7), w.acc_m, 0,
                                                   0, 0);
}

// ---------------------------------------------------------------------------
// V scale on the P side (PS). When a pass's query heads times the head's V groups
// fit the 16 MFMA columns (gs * G <= 16, G <= 4), column n stands for query head
// n % gs and V group n / gs: the S^T product computes every query's scores once
// per group it will meet (the columns were padding), and the PV operand of column
// n is w * s[t, group(n)] -- the token's V scale folded into its weight -- so the
// V operand is the codes alone, exact and unscaled:
//   O^T[d, n] += codes[t, d]^T . (w * s)[t, n]          (16x16x16, hi then lo part)
//   M[n]      += sum_t w[t] * m[t, group(n)]            (fp32 FMAs, per lane)
// Of the output, row d of column n is real where group(d) == group(n): lane (c, n)
// holds rows 4c .. 4c + 3, all in group c * G / 4, so the lanes with n / gs ==
// c * G / 4 write their column's query, those rows' channels, plus M.
// w = 2^k * exp2(x * scale - m_run) with the tier's shift k (INT8 6, INT4 2, INT2
// 0): a weight near the row max times a typical V scale then sits in fp16's
// normal range with room below for its lo part (lo = w * s - hi, normal down to
// w * s = 2^-3), and w * s < 2^15 while s < 2^(7 - k) (w <= 2^(8 + k) under the
// lazy rescale). A tile with a larger scale rescales exactly (w <= 2^k), which
// keeps w * s finite for every finite fp16 V. The stored running max is m_run - k,
// so partial rows of any tier combine as plain log-sum-exp partials.
// ---------------------------------------------------------------------------
template <int BITS>
constexpr int ps_shift() { return BITS == 8 ? 6 : (BITS == 4 ? 2 : 0); }
__device__ __forceinline__ int ps_shift_of(int bits) { return bits == 8 ? 6 : (bits == 4 ? 2 : 0); }
// PS: column n's V group is n / gs (the padding columns past gs * G read group 0).
__device__ __forceinline__ int ps_group(const DecodeArgs& a, int G, int n) {
  const int g = n / a.gs;
  return g < G ? g : 0;
}


// Online-softmax update and PV for PS. kk: the kernel's shift (the weights' unit);
// kb: the shift of the tile's tier (its codes and scales); the generic path's
// tiles of another tier scale the codes by 2^(kk - kb) and the P operand by
// 2^(kb - kk), so the product stays in the kernel's unit.
template <int D, bool QLO, int BITS, int VW>
__device__ __forceinline__ void softmax_pv_ps(Wave<D, QLO>& w, const float* x, const VTile<VW>& vt, int kk, int kb) {
  const VStats& vs = vt.st;
  const float mt = rows_max(vmax(vmax3(x[0], x[1], x[2]), x[3])) * w.scale;
  const float m_new = vmax(w.m_run, mt);
  // The largest V scale of the lane's tokens, as fp16 bits (positive: ordered like
  // the values; a negative or NaN pattern reads as large, which only rescales).
  const uint32_t s2 = __builtin_elementwise_max(h2u(vs.s01) & 0xFFFFu, h2u(vs.s23) & 0xFFFFu);
  const uint32_t s3 = __builtin_elementwise_max(h2u(vs.s01) >> 16, h2u(vs.s23) >> 16);
  const bool big = __builtin_elementwise_max(s2, s3) >= ((uint32_t)(15 + 7 - kb) << 10);
  if (__builtin_amdgcn_ballot_w64(m_new > w.m_run + (big ? 0.f : kLazyRescale))) {
    const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_new);  // m_run = -inf at the start: 0
    w.l_lane *= alpha;
#pragma unroll
    for (int j = 0; j < Wave<D, QLO>::CPM; ++j) w.acc[j] *= alpha;
    w.acc_ml *= alpha;
    w.m_run = m_new;
  }
  const float off = (float)kk - w.m_run;
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], w.scale, off));
  w.l_lane += (p[0] + p[1]) + (p[2] + p[3]);
  const _Float16 sv[4] = {vs.s01[0], vs.s01[1], vs.s23[0], vs.s23[1]};
  const _Float16 mv[4] = {vs.m01[0], vs.m01[1], vs.m23[0], vs.m23[1]};
  const float sc = kb == kk ? 1.f : __builtin_amdgcn_exp2f((float)(kb - kk));  // exact power of two
  float b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w.acc_ml = __builtin_fmaf(p[i], (float)mv[i], w.acc_ml);
    b[i] = __builtin_fmaf((float)sv[i], kb == kk ? p[i] : p[i] * sc, 0.f);
  }
  // b = hi + lo in fp16: hi rounded once, lo the exact remainder rounded once.
  const h4_t bh = {(_Float16)b[0], (_Float16)b[1], (_Float16)b[2], (_Float16)b[3]};
  h4_t bl;
#pragma unroll
  for (int i = 0; i < 4; ++i) bl[i] = (_Float16)__builtin_fmaf((float)bh[i], -1.f, b[i]);
  h4_t va[Wave<D, QLO>::CPM];
  v_codes<BITS, Wave<D, QLO>::CPM, VW>(vt.w, va);
  if (kb != kk) {  // generic-path tile of another tier: codes * 2^(kk - kb), exact
    const _Float16 f = (_Float16)__builtin_amdgcn_exp2f((float)(kk - kb));
    const h4_t f4 = {f, f, f, f};
#pragma unroll
    for (int j = 0; j < Wave<D, QLO>::CPM; ++j) va[j] *= f4;
  }
#pragma unroll
  for (int j = 0; j < Wave<D, QLO>::CPM; ++j) {
    w.acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va[j], bh, w.acc[j], 0, 0, 0);
    w.acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va[j], bl, w.acc[j], 0, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// Generic register path: a tile of a block stored at another tier than the
// kernel's (or whose chunk table names a chunk out of range), including its
// open K group. Rare: only blocks demoted or downgraded under pool pressure.
// ---------------------------------------------------------------------------
// NC codes (4, 8, 16 or 32) of `bits` bits at p (little-endian within bytes),
// one byte each, in out[NC / 4].
template <int NC>
__device__ __forceinline__ void load_as_bytes(const uint8_t* p, int bits, uint32_t* out) {
  if (bits == 8) {
    load_bytes<NC>(p, out);
  } else if (bits == 4) {
    constexpr int NW = NC / 8 > 0 ? NC / 8 : 1;
    uint32_t x[NW];
    load_bytes<NC / 2>(p, x);
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const uint32_t lo = x[i] & 0x0F0F0F0Fu, hi = (x[i] >> 4) & 0x0F0F0F0Fu;  // even / odd codes
      out[2 * i] = perm(hi, lo, 0x05010400u);                                   // codes 8i .. 8i+3
      if (2 * i + 1 < NC / 4) out[2 * i + 1] = perm(hi, lo, 0x07030602u);        // codes 8i+4 .. 8i+7
    }
  } else {
    constexpr int NW = NC / 16 > 0 ? NC / 16 : 1;
    uint32_t x[NW];
    if constexpr (NC >= 16) load_bytes<NC / 4>(p, x);
    else if constexpr (NC == 8) x[0] = *(const uint16_t*)p;
    else x[0] = *p;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const uint32_t y0 = x[i] & 0x03030303u, y1 = (x[i] >> 2) & 0x03030303u;
      const uint32_t y2 = (x[i] >> 4) & 0x03030303u, y3 = (x[i] >> 6) & 0x03030303u;
#pragma unroll
      for (int b = 0; b < 4; ++b) {  // byte b of y_k = code 4b + k
        if (4 * i + b < NC / 4) {
          const uint32_t sel = 0x04000400u | (uint32_t)b | ((uint32_t)b << 8) | ((uint32_t)b << 16) | ((uint32_t)b << 24);
          const uint32_t t01 = perm(y1, y0, sel);  // y0.b, y1.b, y0.b, y1.b
          const uint32_t t23 = perm(y3, y2, sel);  // y2.b, y3.b, y2.b, y3.b
          out[4 * i + b] = perm(t23, t01, 0x05040100u);
        }
      }
    }
  }
}

// One 16-token tile [t0, t0 + 16) of block `blk` stored at `bits` (any tier):
// codes are widened to bytes and go through the 8-bit math. tokens >= n_valid
// are masked; in_res: the tile is the block's open K group (K from the residual,
// head h's channels from element rh of a row).
// The block header is read once and each part's loads issue together: the tile
// is a few memory round trips, not one per row.
template <int D, bool QLO, bool PS>
__device__ __forceinline__ void tile_any(const Wave<D, QLO>& w, const DecodeArgs& a, long blk, int t0, int n_valid,
                                         long rslot, bool in_res, int h, long rh, int lane, int bits, float* x,
                                         VTile<D / 64>& vt) {
  using W = Wave<D, QLO>;
  constexpr int CPL = W::CPL, NQK = W::NQK, CPM = W::CPM;
  const Lay& L = a.L;
  const int c = lane >> 4, n = lane & 15;
  const uint8_t* pages = a.pages;
  const long side = (long)L.H * D * bits / 8;
  const long headb = (long)h * (D * bits / 8);
  const Hdr hd = load_hdr(pages, L, blk);

  // ---- S^T = K Q'^T (+ bias) -------------------------------------------
  f4_t s = {0.f, 0.f, 0.f, 0.f};
  if (in_res) {
    if (a.res.dtype == ECHOKV_F16) s_from_residual<D, QLO, ECHOKV_F16>(w, a, rslot, t0, rh, lane, s);
    else if (a.res.dtype == ECHOKV_BF16) s_from_residual<D, QLO, ECHOKV_BF16>(w, a, rslot, t0, rh, lane, s);
    else s_from_residual<D, QLO, ECHOKV_F32>(w, a, rslot, t0, rh, lane, s);
  } else {
    const long e0 = ((long)(t0 / L.KG) * L.H + h) * D + c * CPL;
    const long rb = row_base_h(L, blk, hd, t0 + n, bits);
    uint32_t kw[CPL / 4];
    load_as_bytes<CPL>(pages + (rb >= 0 ? rb + headb + (long)c * (CPL * bits / 8) : blk * L.stride), bits, kw);
    if (rb < 0) {
#pragma unroll
      for (int i = 0; i < CPL / 4; ++i) kw[i] = 0;
    }
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      uint32_t ks[4], km[4];
      load_bytes<16>(pages + blk * L.stride + L.o_ks + 2 * e0 + 16 * j, ks);
      load_bytes<16>(pages + blk * L.stride + L.o_km + 2 * e0 + 16 * j, km);
      s_block<D, QLO, 0>(w, ks, km, kfrag_bytes(kw + 2 * j), j, s);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = s[i];
    x[i] = (t0 + 4 * c + i < n_valid) ? v : -__builtin_inff();
  }

  // ---- V fragments: tokens t0+4c+i, channels n*CPM + j -------------------
  constexpr int VW = CPM / 4;  // words per token of the lane's V slice, one byte per code
  uint32_t (&vw)[4][VW] = vt.w;
  const int G = D / L.VG;
  const int g = PS ? ps_group(a, G, n) : (n * CPM) / L.VG;
  _Float16 sv[4], mv[4];
  // The four rows at a compile-time width (one branch on the tier, not one per
  // row), so their loads issue together.
  auto load_v = [&](auto width) {
    constexpr int BB = decltype(width)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tv = t0 + 4 * c + i;
      const long rb = row_base_h(L, blk, hd, tv, BB);
      // Every lane loads (a row without a chunk reads its page's first bytes
      // instead), and the masked rows are zeroed after: no branch per row, so
      // the rows' loads issue back to back.
      const long vb = rb >= 0 ? rb + side + headb + (long)n * (CPM * BB / 8) : blk * L.stride;
      load_as_bytes<CPM>(pages + vb, BB, vw[i]);
      const long e = ((long)tv * L.H + h) * G + g;  // tv < block size: inside the page's stats
      sv[i] = *f16p(pages, blk * L.stride + L.o_vs + 2 * e);
      mv[i] = *f16p(pages, blk * L.stride + L.o_vm + 2 * e);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tv = t0 + 4 * c + i;
      if (tv >= n_valid || row_base_h(L, blk, hd, tv, BB) < 0) {
#pragma unroll
        for (int k = 0; k < VW; ++k) vw[i][k] = 0;
        sv[i] = (_Float16)0.f;
        mv[i] = (_Float16)0.f;
      }
    }
  };
  if (bits == 8) load_v(std::integral_constant<int, 8>{});
  else if (bits == 4) load_v(std::integral_constant<int, 4>{});
  else load_v(std::integral_constant<int, 2>{});
  vt.st = VStats{{sv[0], sv[1]}, {sv[2], sv[3]}, {mv[0], mv[1]}, {mv[2], mv[3]}};
}

// ---------------------------------------------------------------------------
// Tier-specialised pipelined path. The 4 waves of a workgroup (the 4 KV heads of
// a head group) stream the split's tiles through one ring of LDS slots,
// filled by direct global->LDS DMA (global_load_lds_dword{,x4}: lane L's bytes
// land at M0 + size * L). A token row holds [K codes of all heads | V codes of
// all heads], so the group's 4 heads are one contiguous 4 * D * b/8-byte
// segment per side: the tile is loaded as whole segments, jobs of 1 KB dealt
// round-robin to the 4 waves, and every wave then reads its own head from LDS.
// (Per-head loads would fetch 64-byte pieces at 1 KB stride: about three times
// the cache-line requests for the same bytes.) Within a DMA job, lane L takes
// 16-byte unit (L + row) % U of its row: the rotation spreads any one head's
// units of the 16 rows over all LDS banks, so the per-head reads are conflict-free.
// The DMAs are issued from inline asm with a 64-bit scalar base (the address
// of the chunk or page being read: pages may span far more than 4 GiB, as in a
// layer view of a pool interleaved across layers) and a 32-bit per-lane byte
// offset within it; the compiler neither sees them nor inserts waits for them. A wave waits with an explicit s_waitcnt vmcnt(n) for
// its own part of the tile about to be read (loads retire in order, so "at most
// n outstanding" covers every older load), then the workgroup meets at a
// barrier: after it every part has landed and every wave is done with the
// previous tile, whose slot the next DMAs then reuse. Every tile issues the
// same number of DMA instructions per wave (a job past the tile's last, or a
// tile the pipelined path does not take, loads 4 dummy bytes from the page
// header into the slot's spare word), so n is a compile-time count.
// ---------------------------------------------------------------------------
#pragma clang diagnostic ignored "-Winline-asm"

// `lds` is wave-uniform; readfirstlane keeps it in a scalar register even where
// the compiler computed it with vector instructions.
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2" ::"v"(off), "s"(__builtin_amdgcn_readfirstlane(lds)),
               "s"(base)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(const uint8_t* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, %2" ::"v"(off), "s"(__builtin_amdgcn_readfirstlane(lds)),
               "s"(base)
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier without a memory fence (a fence would wait for the DMAs in
// flight); the wave's own LDS reads are complete first.
__device__ __forceinline__ void wg_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Half-heads (DecodeArgs::pair): waves 2k and 2k + 1 of a workgroup hold the two
// channel halves of one KV head and so each the partial scores of its half. Each
// adds the other's through LDS: a + b == b + a in IEEE arithmetic, so both waves
// hold the same scores and run the same softmax. Two buffers, alternated by the
// exchange count xi: a wave writes buffer xi & 1 only after the barrier of
// exchange xi - 1, which its partner meets only once its read of exchange xi - 2
// (the same buffer) has returned. Every wave of the workgroup takes part in every
// exchange (the barrier is the workgroup's).
constexpr int kPairLds = 2 * 4 * 4 * 64 * 4;  // [buffer][wave][score][lane] float32
__device__ __forceinline__ void pair_scores(uint8_t* xch, int& xi, int wv, int lane, float* x) {
  float* buf = (float*)xch + (xi & 1) * (4 * 4 * 64);
  ++xi;
#pragma unroll
  for (int i = 0; i < 4; ++i) buf[(wv * 4 + i) * 64 + lane] = x[i];
  wg_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = x[i] + buf[((wv ^ 1) * 4 + i) * 64 + lane];
}

template <int D, int BITS>
struct Ring {
  static constexpr int KB = D * BITS / 8;        // code bytes per token, one side, one head
  static constexpr int U = 4 * KB / 16;          // 16-byte units of the group's segment of a row, one side
  static constexpr int RPI = 64 / U;             // rows per DMA job
  static constexpr int NK = 16 / RPI;            // DMA jobs per side
  static constexpr int SIDE = 16 * 4 * KB;       // one side of a tile, 4 heads
  static constexpr int OFF_V = SIDE;             // K codes | V codes | k_scale, k_min (4 heads) | V scale, V min
  static constexpr int OFF_KS = 2 * SIDE;
  static constexpr int OFF_VS = OFF_KS + 2 * 4 * D * 2;
  static constexpr int OFF_DUMMY = OFF_VS + 2 * 16 * 4 * 4 * 2;  // V stats for G <= 4 groups
  static constexpr int SLOT = OFF_DUMMY + 16;
  static constexpr int J = 2 * NK + 3;           // DMA jobs per tile
  static constexpr int M = (J + 3) / 4;          // DMA instructions per wave per tile
  static_assert(U >= 4 && U <= 64, "segment units");
};

// Ring slots of a workgroup: two-tile steps (PSV 2) take a pair of slots per step,
// with one step in flight while a step computes.
template <int BITS, int PSV>
constexpr int ring_slots() { return PSV == 2 ? 4 : (BITS == 8 ? 3 : 4); }

// LDS byte offset (within a slot's side) of 16-byte unit u of token n.
template <int D, int BITS>
__device__ __forceinline__ uint32_t unit_pos(int n, int u) {
  using R = Ring<D, BITS>;
  return (uint32_t)((n / R::RPI) * 1024 + ((n % R::RPI) * R::U + ((u - n) % R::U + R::U) % R::U) * 16);
}

// Per-block facts of the split's next <= 64 blocks, one block per lane: 64-bit
// byte offsets (from the layer's pages) of the block's page and of its chunks
// (chunk 0 is in the block's own page), tier and residual mapping.
struct BlockLane {
  uint64_t pg, cb1, cb2, cb3;
  int blk;    // -1: not a valid block id
  int tier;
  // kNotFast unless the block is stored at the kernel's tier with every chunk it
  // needs in range; else the K group read from the residual (-1: none), whose
  // tile takes K from the residual. Derived from the loads (not a loaded register
  // itself), so the compiler waits for them once, before the tile loop, rather
  // than with a vmcnt(0) -- which would drain the DMA ring -- at a use inside it.
  int fast_rg;
  int rslot, rgrp;
};
constexpr int kNotFast = -0x7fffffff;

template <int BITS>
__device__ __forceinline__ BlockLane load_block(const DecodeArgs& a, long blk) {
  const Lay& L = a.L;
  BlockLane b{0, 0, 0, 0, -1, 2, kNotFast, -1, -1};
  if (blk < 0 || blk >= L.nb) return b;
  const uint64_t pg = (uint64_t)blk * (uint64_t)L.stride;
  const uint4 hd = *(const uint4*)(a.pages + pg);
  b.blk = (int)blk;
  b.pg = pg;
  b.tier = tier_of(hd.x & 0xffu);
  const uint32_t ids[3] = {hd.y, hd.z, hd.w};
  uint64_t cbs[3];
  bool ok = true;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const uint32_t id = ids[j];
    const uint32_t page = a.kc_mul ? __umulhi(id, a.kc_mul) : id;
    const uint32_t slot = id - page * (uint32_t)L.KC;
    const bool in = (int)id >= 0 && (long)page < L.nb;
    cbs[j] = in ? (uint64_t)page * (uint64_t)L.stride + (uint64_t)L.o_data + (uint64_t)slot * (uint64_t)L.cb
                : pg + (uint64_t)L.o_data;
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

// Per-lane constants of the pipelined path: LDS read offsets within a slot
// for the wave's head (wv, 0..3 within the group).
// 16-byte LDS units of one lane's K slice (D/4 channels of one token): INT8 D/64,
// the narrower tiers fit one unit.
template <int D, int BITS>
constexpr int k_units() { return BITS == 8 ? D / 64 : 1; }

template <int D, int BITS>
struct LaneConst {
  uint32_t k_rd[k_units<D, BITS>()];  // K codes of token n, channels c * D/4 .. (one offset per 16-byte unit)
  uint32_t v_rd[4];                  // V codes of tokens 4c + i, the lane's CPM channels
  uint32_t s_rd;                     // k_scale (k_min at + 4 * D * 2)
  uint32_t vs_rd;                    // V scale of token 4c (32-byte rows: token 4c + i at + 32 i, V min at + 512)
};

template <int D, int BITS, bool PS>
__device__ __forceinline__ LaneConst<D, BITS> lane_const(const DecodeArgs& a, int wv, int lane) {
  using R = Ring<D, BITS>;
  constexpr int CPL = D / 4, CPM = D / 16, VB = CPM * BITS / 8;
  const int c = lane >> 4, n = lane & 15;
  LaneConst<D, BITS> k;
  const int kbyte = wv * R::KB + c * (CPL * BITS / 8);  // within the group's segment
#pragma unroll
  for (int e = 0; e < k_units<D, BITS>(); ++e) k.k_rd[e] = unit_pos<D, BITS>(n, kbyte / 16 + e) + (kbyte % 16);
  const int vbyte = wv * R::KB + n * VB;
#pragma unroll
  for (int i = 0; i < 4; ++i) k.v_rd[i] = R::OFF_V + unit_pos<D, BITS>(4 * c + i, vbyte / 16) + (vbyte % 16);
  k.s_rd = (uint32_t)(R::OFF_KS + wv * D * 2 + 2 * c * CPL);
  const int G = D >> a.vg_shift;
  const int g = PS ? ps_group(a, G, n) : (n * CPM) >> a.vg_shift;
  k.vs_rd = (uint32_t)(R::OFF_VS + 4 * c * 32 + (wv * G + g) * 2);  // 32 bytes per token
  return k;
}

// The DMA jobs of a tile (16 tokens of head group hg) are dealt to the waves:
// wave wv takes jobs wv, wv + 4, ... Each job's per-lane source offset does
// not depend on the tile, only on the job, the lane and the head group, so it
// is computed once per work item (JobLane); a tile adds a wave-uniform base.
// A lane whose unit belongs to a head past the last (H not a multiple of 4)
// loads the same unit of the last head instead: the bytes land in the slot of
// a wave that computes nothing, and every address stays in the layer's pages.
// Code rows: job jj of a side covers rows jj * RPI .. + RPI - 1 of the tile,
// which lie in one chunk (RPI <= tokens per chunk for D >= 64).
template <int D, int BITS>
struct JobLane {
  uint32_t off[Ring<D, BITS>::M];
};

template <int D, int BITS>
__device__ __forceinline__ JobLane<D, BITS> job_lane(const DecodeArgs& a, int wv, int hg, int lane) {
  using R = Ring<D, BITS>;
  static_assert(D >= 64, "a code-row job must not straddle two chunks");
  const Lay& L = a.L;
  const uint32_t rowb = (uint32_t)(2 * D * BITS / 8) * (uint32_t)L.H;
  const int h0 = hg * 4, hl = L.H - 1;
  const int G = D >> a.vg_shift;
  JobLane<D, BITS> jl;
#pragma unroll
  for (int m = 0; m < R::M; ++m) {
    const int j = wv + 4 * m;  // wave-uniform
    uint32_t off = 0;
    if (j < 2 * R::NK) {  // codes: RPI rows of one side
      const int side = j >= R::NK;
      const int jj = side ? j - R::NK : j;
      const int ri = lane / R::U;
      const int t = jj * R::RPI + ri;           // token within the tile
      const int u = (lane % R::U + t) % R::U;  // unit of the segment this lane loads
      const int hu = h0 + (u * 16) / R::KB;
      const int hh = hu < hl ? hu : hl;
      off = (uint32_t)ri * rowb + (side ? rowb / 2 : 0u) + (uint32_t)(hh * R::KB + (u * 16) % R::KB);
    } else if (j < 2 * R::NK + 2) {  // k_scale, then k_min, of the 4 heads
      const int hu = h0 + (16 * lane) / (2 * D);
      const int hh = hu < hl ? hu : hl;
      off = (uint32_t)((j - 2 * R::NK) ? L.o_km : L.o_ks) + (uint32_t)(hh * D * 2 + (16 * lane) % (2 * D));
    } else if (j < R::J) {  // V scale then V min: 2 lanes of 16 bytes per token (32-byte rows in LDS)
      const int arr = lane / 32, t = (lane % 32) / 2;
      const int piece = G == 4 ? lane % 2 : 0;  // G == 2: 16 bytes per token, the odd lane repeats it
      const int hu = h0 + (piece * 16) / (2 * G);
      const int hh = hu < hl ? hu : hl;
      off = (uint32_t)(arr ? L.o_vm : L.o_vs) + (uint32_t)((t * L.H + hh) * G * 2 + (piece * 16) % (2 * G));
    }
    jl.off[m] = off;
  }
  return jl;
}

// Wave WV's share of the DMAs of one tile (16 tokens from block offset t0)
// into ring slot `slot`; the wave's jobs are compile-time, so the per-tile work
// is a few scalar operations per DMA (its 64-bit base) and no vector ones: the
// per-lane offsets are the item's. pg / cb: the block's page and chunk byte
// offsets (wave-uniform); a tile the pipelined path does not take (fast false)
// issues only dummies.
template <int D, int BITS, int WV>
__device__ __forceinline__ void issue_tile_w(const DecodeArgs& a, const JobLane<D, BITS>& jl, uint32_t slot, bool fast,
                                             int t0, int lane, uint64_t pg, uint64_t cb1, uint64_t cb2, uint64_t cb3) {
  using R = Ring<D, BITS>;
  const Lay& L = a.L;
  constexpr int LB = BITS == 8 ? 3 : (BITS == 4 ? 2 : 1);
  const int tpc_shift = a.bs_shift + 1 - LB;  // tokens per chunk = 2 * BS / BITS
  const uint32_t rowb = (uint32_t)(2 * D * BITS / 8) * (uint32_t)L.H;
  const int G = D >> a.vg_shift;
#pragma unroll
  for (int m = 0; m < R::M; ++m) {
    constexpr int j0 = WV;
    const int j = j0 + 4 * m;  // compile-time after unrolling
    if (!fast || j >= R::J) {
      if (lane == 0) dma4(a.pages + pg, 0u, slot + R::OFF_DUMMY);
      continue;
    }
    if (j < 2 * R::NK) {
      const int side = j >= R::NK;
      const int jj = side ? j - R::NK : j;
      const uint32_t tr = (uint32_t)(t0 + jj * R::RPI);  // the job's first token in the block
      const uint32_t ch = tr >> tpc_shift;
      uint64_t cb = pg + (uint64_t)L.o_data;
      if constexpr (BITS >= 4) cb = ch == 1 ? cb1 : cb;
      if constexpr (BITS == 8) cb = ch == 2 ? cb2 : (ch == 3 ? cb3 : cb);
      const uint64_t base = cb + (uint64_t)((tr & ((1u << tpc_shift) - 1)) * rowb);
      dma16(a.pages + base, jl.off[m], slot + (side ? R::OFF_V : 0) + 1024 * jj);
    } else if (j < 2 * R::NK + 2) {
      const uint64_t base = pg + (uint64_t)(((t0 >> a.kg_shift) * L.H) * D * 2);
      if (lane < D / 2) dma16(a.pages + base, jl.off[m], slot + R::OFF_KS + (j - 2 * R::NK) * 4 * D * 2);
    } else {
      const uint64_t base = pg + (uint64_t)(t0 * L.H * G * 2);
      dma16(a.pages + base, jl.off[m], slot + R::OFF_VS);
    }
  }
}

template <int D, int BITS>
__device__ __forceinline__ void issue_tile(const DecodeArgs& a, const JobLane<D, BITS>& jl, uint32_t slot, bool fast,
                                           int t0, int lane, int wv, uint64_t pg, uint64_t cb1, uint64_t cb2,
                                           uint64_t cb3) {
  switch (wv) {
    case 0: issue_tile_w<D, BITS, 0>(a, jl, slot, fast, t0, lane, pg, cb1, cb2, cb3); break;
    case 1: issue_tile_w<D, BITS, 1>(a, jl, slot, fast, t0, lane, pg, cb1, cb2, cb3); break;
    case 2: issue_tile_w<D, BITS, 2>(a, jl, slot, fast, t0, lane, pg, cb1, cb2, cb3); break;
    default: issue_tile_w<D, BITS, 3>(a, jl, slot, fast, t0, lane, pg, cb1, cb2, cb3); break;
  }
}

// One pipelined tile from LDS slot `sp` (tier BITS, K from codes): its scores
// (log2 units, masked past n_rel valid tokens) and V fragments.
template <int D, bool QLO, int BITS>
__device__ __forceinline__ void compute_tile(const Wave<D, QLO>& w, const DecodeArgs& a, const LaneConst<D, BITS>& k,
                                             const uint8_t* sp, int n_rel, int lane, float* x,
                                             VTile<(D / 16 * BITS / 8 >= 4 ? D / 16 * BITS / 8 / 4 : 1)>& vt) {
  using W = Wave<D, QLO>;
  using R = Ring<D, BITS>;
  constexpr int CPL = W::CPL, NQK = W::NQK, CPM = W::CPM;
  const int c = lane >> 4;
  constexpr int KW = CPL * BITS / 32 > 0 ? CPL * BITS / 32 : 1;
  uint32_t kw[KW];
  static_assert(BITS != 8 || KW == 4 * k_units<D, BITS>(), "INT8 K slice: whole 16-byte units");
  if constexpr (BITS == 8) {
#pragma unroll
    for (int e = 0; e < k_units<D, BITS>(); ++e) load_bytes<16>(sp + k.k_rd[e], kw + 4 * e);
  } else {
    load_bytes<CPL * BITS / 8>(sp + k.k_rd[0], kw);
  }
  constexpr int VB = CPM * BITS / 8;
  constexpr int VW = VB >= 4 ? VB / 4 : 1;
  uint32_t (&vw)[4][VW] = vt.w;
#pragma unroll
  for (int i = 0; i < 4; ++i) load_bytes<VB>(sp + k.v_rd[i], vw[i]);
  // V scale / min of the lane's 4 tokens: 32-byte rows per token, scales then mins.
  const _Float16* vs = (const _Float16*)(sp + k.vs_rd);
  h2_t s01 = {vs[0], vs[16]}, s23 = {vs[32], vs[48]};
  h2_t m01 = {vs[256], vs[272]}, m23 = {vs[288], vs[304]};

  f4_t s = {0.f, 0.f, 0.f, 0.f};
  const CodeK ck = code_consts<BITS>();
  // k_scale / k_min words one 32-channel block ahead of their use, so each
  // block's LDS reads are in flight under the previous block's MFMAs.
  uint32_t ks[2][4], km[2][4];
  load_bytes<16>(sp + k.s_rd, ks[0]);
  load_bytes<16>(sp + k.s_rd + 4 * D * 2, km[0]);
#pragma unroll
  for (int j = 0; j < NQK; ++j) {
    if (j + 1 < NQK) {
      load_bytes<16>(sp + k.s_rd + 16 * (j + 1), ks[(j + 1) & 1]);
      load_bytes<16>(sp + k.s_rd + 4 * D * 2 + 16 * (j + 1), km[(j + 1) & 1]);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the next block's reads above this block's math
    s_block<D, QLO, BITS>(w, ks[j & 1], km[j & 1], kfrag_j<BITS>(kw, j, ck), j, s);
  }
  // Tokens past the sequence (the block's last tile) get p = 0 and V = 0: their
  // page bytes are arbitrary and 0 * inf would poison the sum. The scores are
  // selected on every tile, before any branch: their first reader must follow
  // the MFMAs in straight-line code, where the compiler places the wait states
  // an MFMA result needs (across a branch it does not, and the max would read
  // an unfinished accumulator).
  const int t = 4 * c;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = t + i < n_rel ? s[i] : -__builtin_inff();
    asm volatile("" : "+v"(x[i]));  // emits nothing; keeps the select here, ahead of the branch
  }
  if (n_rel < 16) {
    const uint32_t k01 = t + 1 < n_rel ? ~0u : (t < n_rel ? 0xFFFFu : 0u);
    const uint32_t k23 = t + 3 < n_rel ? ~0u : (t + 2 < n_rel ? 0xFFFFu : 0u);
    s01 = u2h(h2u(s01) & k01);
    m01 = u2h(h2u(m01) & k01);
    s23 = u2h(h2u(s23) & k23);
    m23 = u2h(h2u(m23) & k23);
  }
  vt.st = VStats{s01, s23, m01, m23};
}

// ---------------------------------------------------------------------------
// Two tiles per step (PS with 4 query heads x 4 V groups, D 128; the INT8 kernel:
// at INT2 / INT4 the step's operands need about 200 registers, so those tiers keep
// one tile per step at three waves per SIMD, which measured faster). Tiles u = 0, 1
// of a step share its fixed costs (one barrier, one softmax reduction, one
// exponent per score), and both contractions use all 16 MFMA columns:
//  S^T: column n = q + 4 (u + 2x) is query q's scores of tile u (x: a copy), so a
//       lane builds the (q * k_scale) hi / lo operand of one tile's K group only;
//       each tile's MFMAs fill every column, and a lane keeps its own tile's.
//  PV:  column n = q + 4g (query q, V group g), as with one tile; K = 32 runs over
//       the lane's 4 tokens of tile 0, then of tile 1, so one 16x16x32 product per
//       16 channels and weight part takes both tiles. The other tile's weights come
//       from the neighbouring group of 4 lanes in the row of 16 (DPP row_ror:4, bank
//       masked): that group is the same query at the other tile.
// ---------------------------------------------------------------------------
constexpr int kRowRor4 = 0x124;  // DPP row_ror:4
template <int BANKS>
__device__ __forceinline__ float dpp_ror4(float old, float src) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(src), kRowRor4, 0xF, BANKS,
                                                    false));
}

// S^T of block j for both tiles: `ks` this lane's own tile's k_scale words (its
// columns' tile), km0 / km1 each tile's k_min words, kf0 / kf1 each tile's codes.
template <int D, bool QLO, int BITS>
__device__ __forceinline__ void s_pair_block(const Wave<D, QLO>& w, const uint32_t* ks, const uint32_t* km0,
                                             const uint32_t* km1, const h8_t& kf0, const h8_t& kf1, int j, f4_t& s0,
                                             f4_t& s1) {
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h2_t q = u2h(w.qn[4 * j + i]), sc = u2h(ks[i]);
    const h2_t ph = q * sc;
    h2_t pl = __builtin_elementwise_fma(q, sc, -ph);
    if constexpr (QLO) pl = __builtin_elementwise_fma(u2h(w.ql[4 * j + i]), sc, pl);
    hi[i] = h2u(ph);
    lo[i] = h2u(pl);
  }
  const h8_t h8 = w2h8(hi[0], hi[1], hi[2], hi[3]), l8 = w2h8(lo[0], lo[1], lo[2], lo[3]);
  const h8_t qh = w2h8(w.qn[4 * j], w.qn[4 * j + 1], w.qn[4 * j + 2], w.qn[4 * j + 3]);
  const h8_t m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f, (_Float16)-1024.0f, (_Float16)-1024.0f,
                      (_Float16)-1024.0f, (_Float16)-1024.0f, (_Float16)-1024.0f, (_Float16)-1024.0f};
  s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf0, h8, s0, 0, 0, 0);
  s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf1, h8, s1, 0, 0, 0);
  s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf0, l8, s0, 0, 0, 0);
  s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf1, l8, s1, 0, 0, 0);
  if constexpr (BITS == 8) {
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(m1024, h8, s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(m1024, h8, s1, 0, 0, 0);
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(m1024, l8, s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(m1024, l8, s1, 0, 0, 0);
  } else {
    (void)m1024;
  }
  s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w2h8(km0[0], km0[1], km0[2], km0[3]), qh, s0, 0, 0, 0);
  s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w2h8(km1[0], km1[1], km1[2], km1[3]), qh, s1, 0, 0, 0);
  if constexpr (QLO) {
    const h8_t ql = w2h8(w.ql[4 * j], w.ql[4 * j + 1], w.ql[4 * j + 2], w.ql[4 * j + 3]);
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w2h8(km0[0], km0[1], km0[2], km0[3]), ql, s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w2h8(km1[0], km1[1], km1[2], km1[3]), ql, s1, 0, 0, 0);
  }
}

// One two-tile step from LDS slots sp0 / sp1 (tier BITS, both tiles taken by the
// pipelined path): n_rel0 / n_rel1 valid tokens in each (16 or fewer). The online
// softmax state is the one-tile PS state (columns q + 4g), so single tiles and
// generic-path tiles mix freely with steps. Phases are kept apart (sched
// barriers) so that each phase's operands alone are live: the K words and S
// accumulators, then the weights, then the V codes half a head at a time.
template <int D, bool QLO, int BITS>
__device__ __forceinline__ void pair_step(Wave<D, QLO>& w, const LaneConst<D, BITS>& k, const uint8_t* sp0,
                                          const uint8_t* sp1, int n_rel0, int n_rel1, int lane) {
  using W = Wave<D, QLO>;
  constexpr int CPL = W::CPL, NQK = W::NQK, CPM = W::CPM;
  constexpr int kk = ps_shift<BITS>();
  static_assert(D == 128, "two-tile steps: 4 query heads x 4 V groups of 32 channels");
  const int c = lane >> 4, n = lane & 15;
  const bool t1 = (n >> 2) & 1;         // the lane's S^T column belongs to tile 1
  const uint8_t* spo = t1 ? sp1 : sp0;  // its own tile's slot (per lane)

  // ---- S^T of both tiles ----
  constexpr int KW = CPL * BITS / 32 > 0 ? CPL * BITS / 32 : 1;
  uint32_t kw0[KW], kw1[KW];
  if constexpr (BITS == 8) {
#pragma unroll
    for (int e = 0; e < k_units<D, BITS>(); ++e) {
      load_bytes<16>(sp0 + k.k_rd[e], kw0 + 4 * e);
      load_bytes<16>(sp1 + k.k_rd[e], kw1 + 4 * e);
    }
  } else {
    load_bytes<CPL * BITS / 8>(sp0 + k.k_rd[0], kw0);
    load_bytes<CPL * BITS / 8>(sp1 + k.k_rd[0], kw1);
  }
  f4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
  const CodeK ck = code_consts<BITS>();
#pragma unroll
  for (int j = 0; j < NQK; ++j) {
    uint32_t ks[4], km0[4], km1[4];
    load_bytes<16>(spo + k.s_rd + 16 * j, ks);
    load_bytes<16>(sp0 + k.s_rd + 4 * D * 2 + 16 * j, km0);
    load_bytes<16>(sp1 + k.s_rd + 4 * D * 2 + 16 * j, km1);
    s_pair_block<D, QLO, BITS>(w, ks, km0, km1, kfrag_j<BITS>(kw0, j, ck), kfrag_j<BITS>(kw1, j, ck), j, s0, s1);
  }
  // The lane's own tile's scores, masked past its valid tokens; selected in
  // straight-line code right after the MFMAs (their first reader must be one the
  // compiler sees, so it places the wait states the MFMA results need).
  const int t = 4 * c;
  const int nr = t1 ? n_rel1 : n_rel0;
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = t + i < nr ? (t1 ? s1[i] : s0[i]) : -__builtin_inff();
    asm volatile("" : "+v"(x[i]));
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- weights: online softmax over both tiles' scores of each query ----
  // V scale / min of the lane's 4 tokens of each tile, its column's V group
  // (32-byte rows per token; tokens past the sequence: 0, their weights are 0).
  const _Float16* vs0 = (const _Float16*)(sp0 + k.vs_rd);
  const _Float16* vs1 = (const _Float16*)(sp1 + k.vs_rd);
  h2_t sa = {vs0[0], vs0[16]}, sb = {vs0[32], vs0[48]}, sc = {vs1[0], vs1[16]}, sd = {vs1[32], vs1[48]};
  h2_t ma = {vs0[256], vs0[272]}, mb = {vs0[288], vs0[304]}, mc = {vs1[256], vs1[272]}, md = {vs1[288], vs1[304]};
  if (n_rel0 < 16 || n_rel1 < 16) {
    auto keep = [&](int nrel, uint32_t& k01, uint32_t& k23) {
      k01 = t + 1 < nrel ? ~0u : (t < nrel ? 0xFFFFu : 0u);
      k23 = t + 3 < nrel ? ~0u : (t + 2 < nrel ? 0xFFFFu : 0u);
    };
    uint32_t a01, a23, b01, b23;
    keep(n_rel0, a01, a23);
    keep(n_rel1, b01, b23);
    sa = u2h(h2u(sa) & a01), ma = u2h(h2u(ma) & a01), sb = u2h(h2u(sb) & a23), mb = u2h(h2u(mb) & a23);
    sc = u2h(h2u(sc) & b01), mc = u2h(h2u(mc) & b01), sd = u2h(h2u(sd) & b23), md = u2h(h2u(md) & b23);
  }
  float mt = rows_max(vmax(vmax3(x[0], x[1], x[2]), x[3]));
  mt = vmax(mt, dpp_ror4<0xF>(mt, mt));
  mt *= w.scale;
  const float m_new = vmax(w.m_run, mt);
  // The largest V scale (fp16 bits; a negative or NaN pattern reads as large).
  const uint32_t sm0 = __builtin_elementwise_max(h2u(sa) & 0xFFFFu, h2u(sb) & 0xFFFFu);
  const uint32_t sm1 = __builtin_elementwise_max(h2u(sa) >> 16, h2u(sb) >> 16);
  const uint32_t sm2 = __builtin_elementwise_max(h2u(sc) & 0xFFFFu, h2u(sd) & 0xFFFFu);
  const uint32_t sm3 = __builtin_elementwise_max(h2u(sc) >> 16, h2u(sd) >> 16);
  const uint32_t smax = __builtin_elementwise_max(__builtin_elementwise_max(sm0, sm1), __builtin_elementwise_max(sm2, sm3));
  const bool big = smax >= ((uint32_t)(15 + 7 - kk) << 10);
  if (__builtin_amdgcn_ballot_w64(m_new > w.m_run + (big ? 0.f : kLazyRescale))) {
    const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_new);
    w.l_lane *= alpha;
#pragma unroll
    for (int j = 0; j < CPM; ++j) w.acc[j] *= alpha;
    w.acc_ml *= alpha;
    w.m_run = m_new;
  }
  const float off = (float)kk - w.m_run;
  float p[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float own = __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], w.scale, off));
    p[i] = dpp_ror4<0xA>(own, own);      // tile 0: odd groups of 4 lanes take the neighbour's
    p[4 + i] = dpp_ror4<0x5>(own, own);  // tile 1: even groups take the neighbour's
  }
  w.l_lane += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  const _Float16 sv[8] = {sa[0], sa[1], sb[0], sb[1], sc[0], sc[1], sd[0], sd[1]};
  const _Float16 mv[8] = {ma[0], ma[1], mb[0], mb[1], mc[0], mc[1], md[0], md[1]};
  float b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    w.acc_ml = __builtin_fmaf(p[i], (float)mv[i], w.acc_ml);
    b[i] = __builtin_fmaf((float)sv[i], p[i], 0.f);
  }
  h8_t bh, bl;
#pragma unroll
  for (int i = 0; i < 8; ++i) bh[i] = (_Float16)b[i];
#pragma unroll
  for (int i = 0; i < 8; ++i) bl[i] = (_Float16)__builtin_fmaf((float)bh[i], -1.f, b[i]);
  __builtin_amdgcn_sched_barrier(0);

  // ---- O^T += V^T P^T over both tiles, half a head's channels at a time ----
  constexpr int VB = CPM * BITS / 8;
  constexpr int VW = VB >= 4 ? VB / 4 : 1;
  uint32_t vw0[4][VW], vw1[4][VW];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    load_bytes<VB>(sp0 + k.v_rd[i], vw0[i]);
    load_bytes<VB>(sp1 + k.v_rd[i], vw1[i]);
  }
  auto pv_half = [&](auto part) {
    constexpr int P = decltype(part)::value;
    h4_t va0[CPM / 2], va1[CPM / 2];
    v_codes_half<BITS, CPM, VW, P>(vw0, va0);
    v_codes_half<BITS, CPM, VW, P>(vw1, va1);
#pragma unroll
    for (int j = 0; j < CPM / 2; ++j) {
      const h8_t av = __builtin_shufflevector(va0[j], va1[j], 0, 1, 2, 3, 4, 5, 6, 7);
      w.acc[P * CPM / 2 + j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh, w.acc[P * CPM / 2 + j], 0, 0, 0);
      w.acc[P * CPM / 2 + j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl, w.acc[P * CPM / 2 + j], 0, 0, 0);
    }
  };
  pv_half(std::integral_constant<int, 0>{});
  pv_half(std::integral_constant<int, 1>{});
}

// Wait for this wave's part of the tile about to be read: `ahead` tiles were
// issued after it (wave-uniform, NB - 2 at most), M DMA instructions each, so at
// most ahead * M of this wave's loads may stay in flight.
template <int M, int K>
__device__ __forceinline__ void wait_ahead(int ahead) {
  if constexpr (K <= 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= K) wait_vmcnt<K * M>();
    else wait_ahead<M, K - 1>(ahead);
  }
}
template <int D, int BITS, int NB>
__device__ __forceinline__ void wait_tile(int ahead) {
  static_assert((NB - 2) * Ring<D, BITS>::M <= 63, "vmcnt holds at most 63");
  wait_ahead<Ring<D, BITS>::M, NB - 2>(ahead);
}

__device__ __forceinline__ uint32_t rl(uint32_t v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ uint64_t rl64(uint64_t v, int lane) {
  return (uint64_t)rl((uint32_t)v, lane) | ((uint64_t)rl((uint32_t)(v >> 32), lane) << 32);
}

// Blocks per split of a sequence of n_blocks blocks:
// max(blocks_per_split, ceil(blocks / num_splits)).
__device__ __forceinline__ int split_blocks(const DecodeArgs& a, int n_blocks) {
  const int per = (n_blocks + a.num_splits - 1) / a.num_splits;
  return a.bps > per ? a.bps : per;
}

__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

// Inclusive prefixes over sequences [s0, s0 + 64), one per lane, of the
// number of splits before the last (bits 7 and up) and of last splits (low 7
// bits: at most 64).
__device__ __forceinline__ int scan_chunk(const DecodeArgs& a, long s0, int lane) {
  const long s = s0 + lane;
  const int len = s < a.num_seqs ? (int)a.lens[s] : 0;
  int x = 0;
  if (len > 0) {
    const int nb = (len + a.L.BS - 1) >> a.bs_shift;
    const int bps = split_blocks(a, nb);
    x = (((nb + bps - 1) / bps - 1) << 7) | 1;
  }
  return wave_incl_scan(x, lane);
}
__device__ __forceinline__ int scan_total(int incl) {
  const int t = __builtin_amdgcn_readlane(incl, 63);
  return (t >> 7) + (t & 127);
}

// The si-th of the batch's non-empty splits, false past the last one. Order:
// every sequence's last split (sequence order), then the others (sequence
// order). A last split is the irregular one -- shorter, and holding the open K
// group, whose tiles take the slower generic path -- so it starts early and
// the work items dispatched last, whose run time is the kernel's tail, are
// the uniform full ones. incl0: scan_chunk of the first 64 sequences.
__device__ __forceinline__ bool locate(const DecodeArgs& a, long si, int lane, int incl0, long& seq, int& split) {
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int shift = pass == 0 ? 0 : 7, mask = pass == 0 ? 127 : -1;
    long base = 0;
    int incl = incl0;
    for (long s0 = 0; s0 < a.num_seqs; s0 += 64) {
      if (s0 > 0) incl = scan_chunk(a, s0, lane);
      const int mine = (incl >> shift) & mask;
      const int tot = __builtin_amdgcn_readlane(mine, 63);
      if (si < base + tot) {
        const int k = __builtin_popcountll(__builtin_amdgcn_ballot_w64(base + mine <= si));
        const int excl = k == 0 ? 0 : __builtin_amdgcn_readlane(mine, k - 1);
        seq = s0 + k;
        if (pass == 1) {
          split = (int)(si - base - excl);
        } else {  // the last split: after the sequence's others
          const int prev_incl = __builtin_amdgcn_readlane(incl, k) >> 7;
          const int prev_excl = k == 0 ? 0 : __builtin_amdgcn_readlane(incl, k - 1) >> 7;
          split = prev_incl - prev_excl;
        }
        return true;
      }
      base += tot;
    }
    si -= base;
  }
  return false;
}

// Where a span's result goes: the normalized output row of the sequence (the span
// is the whole sequence), or unnormalized partials (acc, and (max, sum) in ml) at
// row part_row0 + qh * part_stride of the workspaces, merged later.
struct SpanSink {
  long part_row0;
  int part_stride;
  bool direct;
  // Balanced schedule: blocks of the workgroup's range after this span, and the
  // range's length (0: no priorities).
  int rem_after, total;
};

// A tier pass (DecodeArgs::tier_mask): which of a span's blocks this kernel takes,
// and whether the span continues the partial result already in its rows.
struct SpanPass {
  bool on;     // false: every valid block (one pass over the layer)
  bool other;  // also blocks whose tier is not in `mask`
  int mask;    // the tiers that have passes (2 | 4 | 8)
  bool carry;  // start from the span's partial row instead of afresh
};

// Wave priority from the share of the workgroup's range still ahead of it: the
// co-resident workgroups of a CU start at different times, and the one with the
// most left issues first, so they finish together instead of in start order.
__device__ __forceinline__ void range_priority(int left, int total) {
  if (4 * left > 3 * total) __builtin_amdgcn_s_setprio(3);
  else if (4 * left > 2 * total) __builtin_amdgcn_s_setprio(2);
  else if (4 * left > total) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// Blocks [b_start, b_end) of sequence `seq` for the KV heads of head group hg
// (one wave per head).
template <int D, int BITS, bool QLO, bool PASSES, bool PAIR, int PS>
__device__ __forceinline__ void decode_span(const DecodeArgs& a, long seq, int b_start, int b_end, int hg, int wv,
                                            int lane, uint8_t* ring, uint32_t ring0, SpanSink sink,
                                            SpanPass pass = SpanPass{false, true, 0, false}) {
  using W = Wave<D, QLO>;
  using R = Ring<D, BITS>;
  constexpr int NB = ring_slots<BITS, PS>();
  static_assert(PS != 2 || (D == 128 && !PAIR), "two-tile steps: D 128, whole heads");
  const Lay& L = a.L;
  const int seq_len = (int)a.lens[seq];
  const long q_row = a.q_rows ? a.q_rows[seq] : seq;
  const long bt_row = a.bt_rows ? a.bt_rows[seq] : seq;
  const int c = lane >> 4, n = lane & 15;
  const int h = hg * kHeadsPerGroup + wv;
  const bool live = h < L.H;  // a wave past the last head still loads its share of every tile
  // Half-heads (PAIR, DecodeArgs::pair): KV head kh = h / 2, channels from half * D of its query
  // and output rows, RD floats per workspace row. A wave past the last head then
  // computes on its slot's bytes too (never written out), so that every wave meets
  // every score exchange; its memory reads use the last head (ha).
  constexpr bool pair = PAIR;
  const int kh = pair ? h >> 1 : h;
  const int half = pair ? h & 1 : 0;
  const int RD = pair ? 2 * D : D;
  const int ha = live ? h : L.H - 1;
  const long rh = pair ? (long)(ha >> 1) * a.res.s2 + (ha & 1) * D : (long)ha * a.res.s2;
  uint8_t* const xch = ring + NB * R::SLOT;  // the score exchange (pair only)
  int xi = 0;
  // Columns: query head qcol of the pass (PS: one per V group, cols = gs * G of them);
  // `mine`: the lane's output rows are real (PS: its rows' V group is its column's).
  const int G = D >> a.vg_shift;
  const int cols = PS ? a.gs * G : a.gs;
  const int qcol = PS ? n % a.gs : n;
  const bool mine = live && n < cols && (!PS || n / a.gs == (c * G) >> 2);
  constexpr int kk = PS ? ps_shift<BITS>() : 0;  // the weights' unit (PS): 2^kk

  W w;
  // The first chunk's block table row is requested with the query, so their
  // round trips overlap; its page headers follow before the query is converted.
  const int nb_first = b_end - b_start < 64 ? b_end - b_start : 64;
  BlockLane bl;
  {
    const bool qv = live && n < cols;
    const long qb = q_row * a.q_s0 + (long)(kh * a.gqa + a.g0 + (qv ? qcol : 0)) * a.q_s1 + half * D + c * W::CPL;
    float xq[W::CPL];
    // Scores are scaled inside the exponent (exp2(s * x - m)); the max is taken
    // on unscaled scores, which needs the scale positive: a negative one flips
    // the query's sign (exact), a zero one becomes 2^-100 (every weight equal,
    // as at zero, and masked scores stay -inf).
    const float q_sign = a.scale_log2 < 0.f ? -1.f : 1.f;
    w.scale = fmaxf(fabsf(a.scale_log2), 7.8886090522101181e-31f);
    if (qv) {
      ld_n<W::CPL>(a.q, a.q_dtype, qb, xq);
    } else {
#pragma unroll
      for (int e = 0; e < W::CPL; ++e) xq[e] = 0.f;
    }
    bl = load_block<BITS>(a, lane < nb_first ? (long)a.bt[bt_row * a.bt_s0 + b_start + lane] : -1L);
#pragma unroll
    for (int i = 0; i < W::CPL / 2; ++i) {
      const float x0 = q_sign * xq[2 * i], x1 = q_sign * xq[2 * i + 1];
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
  w.acc_m = f4_t{0.f, 0.f, 0.f, 0.f};
  w.acc_ml = 0.f;
  w.m_run = -__builtin_inff();
  w.l_lane = 0.f;
  // A later tier pass continues the partial result the passes before it left in
  // the span's row (its sum in one lane of the column, so the cross-row sum
  // restores it), loaded once the span has a block of this pass's tier; a span
  // with none leaves its row as it is.
  bool carried = !pass.carry;
  auto load_carry = [&]() {
    if (live && n < cols) {
      const long row = sink.part_row0 + ((long)kh * a.gqa + a.g0 + qcol) * sink.part_stride;
      const float* src = a.acc + row * RD + half * D;
      if (mine) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int j = 0; j < W::CPM; ++j) w.acc[j][i] = src[(4 * c + i) * W::CPM + j];
        }
      }
      w.m_run = a.ml[row * 2] + (float)kk;  // stored: m_run - kk
      w.l_lane = c == 0 ? a.ml[row * 2 + 1] : 0.f;
    }
    carried = true;
  };

  const LaneConst<D, BITS> kc = lane_const<D, BITS, PS != 0>(a, wv, lane);
  const JobLane<D, BITS> jl = job_lane<D, BITS>(a, wv, hg, lane);
  const int tpb_shift = a.bs_shift - 4;  // tiles per block = BS / 16
  const bool stats_ok = (D >> a.vg_shift) == 2 || (D >> a.vg_shift) == 4;
  for (int c0 = b_start; c0 < b_end; c0 += 64) {
    const int nb = b_end - c0 < 64 ? b_end - c0 : 64;
    if (c0 != b_start) bl = load_block<BITS>(a, lane < nb ? (long)a.bt[bt_row * a.bt_s0 + c0 + lane] : -1L);
    // PASSES: the blocks this kernel takes, moved to the front of the chunk's
    // lanes in order, so the tile loop runs over them alone; b_orig keeps each
    // one's place in the sequence. (Already in front -- every valid block of a
    // one-pass launch, or of a layer stored at one tier -- they stay where they
    // are.) Without PASSES every block keeps its lane and invalid ones are skipped.
    int b_orig = lane;
    int n_take = nb;
    uint64_t m_blk = ~0ull;
    if constexpr (!PASSES) {
      m_blk = __builtin_amdgcn_ballot_w64(bl.blk >= 0);
    } else {
      const bool take = bl.blk >= 0 && (!pass.on || bl.tier == BITS || (pass.other && !(pass.mask & bl.tier)));
      const uint64_t m_take = __builtin_amdgcn_ballot_w64(take);
      n_take = __builtin_popcountll(m_take);
      if (m_take != (n_take == 64 ? ~0ull : (1ull << n_take) - 1)) {
        const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m_take >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)m_take, 0u));
        const int to = 4 * (take ? below : n_take + (lane - below));  // a permutation of the lanes
        auto push = [&](uint32_t v) { return (uint32_t)__builtin_amdgcn_ds_permute(to, (int)v); };
        auto push64 = [&](uint64_t v) { return (uint64_t)push((uint32_t)v) | ((uint64_t)push((uint32_t)(v >> 32)) << 32); };
        bl.pg = push64(bl.pg);
        if constexpr (BITS >= 4) bl.cb1 = push64(bl.cb1);
        if constexpr (BITS == 8) {
          bl.cb2 = push64(bl.cb2);
          bl.cb3 = push64(bl.cb3);
        }
        bl.blk = (int)push((uint32_t)bl.blk);
        bl.tier = (int)push((uint32_t)bl.tier);
        bl.fast_rg = (int)push((uint32_t)bl.fast_rg);
        bl.rslot = (int)push((uint32_t)bl.rslot);
        bl.rgrp = (int)push((uint32_t)bl.rgrp);
        b_orig = (int)push((uint32_t)lane);
      }
    }
    // Every taken block but the sequence's last is full; the last one taken may be it.
    const int last_b = !PASSES ? nb - 1 : (n_take > 0 ? (int)rl((uint32_t)b_orig, n_take - 1) : 0);
    const int last_n = seq_len - (c0 + last_b) * L.BS < L.BS ? seq_len - (c0 + last_b) * L.BS : L.BS;
    const int n_tiles = n_take > 0 ? ((n_take - 1) * L.BS + last_n + 15) >> 4 : 0;
    auto orig = [&](int b) { return PASSES ? (int)rl((uint32_t)b_orig, b) : b; };
    if (PASSES && !carried && n_take > 0) load_carry();

    // A tile takes the pipelined path when its block is stored at the kernel's
    // tier with every chunk in range and it is not the block's open K group;
    // the others (rare: demoted / downgraded blocks, each sequence's open
    // group) are computed on the generic path from global memory (generic_tiles).
    // Per-block bit masks (one bit per lane = block) keep the per-tile test scalar.
    const uint64_t m_fast = stats_ok ? __builtin_amdgcn_ballot_w64(lane < n_take && bl.fast_rg != kNotFast) : 0ull;
    const uint64_t m_open = __builtin_amdgcn_ballot_w64(bl.fast_rg >= 0);
    auto piped = [&](int tt) -> bool {
      const int b = tt >> tpb_shift;
      if (!((m_fast >> b) & 1)) return false;
      if (!((m_open >> b) & 1)) return true;
      const int t0 = (tt & ((1 << tpb_shift) - 1)) << 4;
      return (int)rl((uint32_t)bl.fast_rg, b) != (t0 >> a.kg_shift);
    };
    auto issue = [&](int tt) {
      const int b = tt >> tpb_shift;
      const int t0 = (tt & ((1 << tpb_shift) - 1)) << 4;
      const uint64_t pg = rl64(bl.pg, b);
      const uint64_t cb1 = BITS >= 4 ? rl64(bl.cb1, b) : 0u;
      const uint64_t cb2 = BITS == 8 ? rl64(bl.cb2, b) : 0u;
      const uint64_t cb3 = BITS == 8 ? rl64(bl.cb3, b) : 0u;
      const uint32_t slot = ring0 + (uint32_t)((tt % NB) * R::SLOT);
      issue_tile<D, BITS>(a, jl, slot, piped(tt), t0, lane, wv, pg, cb1, cb2, cb3);
    };

    constexpr int VW = W::CPM * BITS / 8 >= 4 ? W::CPM * BITS / 8 / 4 : 1;
    // One pipelined tile on its own (the one-tile loop; a step whose other tile
    // is not taken).
    auto single = [&](int tt) {
      const int b = tt >> tpb_shift;
      const int t0 = (tt & ((1 << tpb_shift) - 1)) << 4;
      const int n_valid = seq_len - ((c0 + orig(b)) << a.bs_shift);
      float x[4];
      VTile<VW> vt;
      compute_tile<D, QLO, BITS>(w, a, kc, ring + (tt % NB) * R::SLOT, n_valid - t0, lane, x, vt);
      if (pair) pair_scores(xch, xi, wv, lane, x);
      if constexpr (PS) softmax_pv_ps<D, QLO, BITS, VW>(w, x, vt, kk, kk);
      else softmax_pv<D, QLO, BITS, VW>(w, x, vt, vscale_mask<BITS>());
    };
    // The chunk's tiles the pipeline does not take (each sequence's open K group,
    // blocks at another tier), on the generic register path. They run right after
    // the pipeline's first DMAs are issued: their loads retire behind those DMAs,
    // so their memory latency overlaps the pipeline's fill instead of adding to the
    // span's end (the workgroups holding an open group are the kernel's last).
    const uint64_t m_valid = (!PASSES ? m_blk : (n_take >= 64 ? ~0ull : (1ull << n_take) - 1)) &
                             (nb >= 64 ? ~0ull : (1ull << nb) - 1);
    auto generic_tiles = [&]() {
      if (!(live || pair) || ((m_valid & ~m_fast) == 0 && (m_valid & m_open) == 0)) return;
#pragma unroll 1
      for (int tt = 0; tt < n_tiles; ++tt) {
        const int b = tt >> tpb_shift;
        const long blk = (int)rl((uint32_t)bl.blk, b);
        if (blk < 0 || piped(tt)) continue;
        const int t0 = (tt & ((1 << tpb_shift) - 1)) << 4;
        const int tier = (int)rl((uint32_t)bl.tier, b);
        const int rgrp = (int)rl((uint32_t)bl.rgrp, b);
        const long rslot = (int)rl((uint32_t)bl.rslot, b);
        const bool in_res = rslot >= 0 && rgrp == (t0 >> a.kg_shift);
        const int n_valid = seq_len - ((c0 + orig(b)) << a.bs_shift);
        float x[4];
        VTile<D / 64> vt;  // codes widened to bytes
        tile_any<D, QLO, PS != 0>(w, a, blk, t0, n_valid, rslot, in_res, ha, rh, lane, tier, x, vt);
        if (pair) pair_scores(xch, xi, wv, lane, x);
        if constexpr (PS)
          softmax_pv_ps<D, QLO, 8, D / 64>(w, x, vt, kk, ps_shift_of(tier));
        else
          softmax_pv<D, QLO, 8, D / 64>(w, x, vt,
                                        tier == 8 ? vscale_mask<8>() : (tier == 4 ? vscale_mask<4>() : vscale_mask<2>()));
      }
    };
    if constexpr (PS == 2) {
      // Two tiles per step: step pp is tiles 2pp, 2pp + 1 in slots of the ring's
      // NB / 2 pairs. Wait for this wave's part of step pp, meet the others (every
      // part has landed; every wave is done with step pp - 1), refill step pp - 1's
      // pair with step pp + NB/2 - 1, compute step pp. A tile past the last of the
      // chunk issues dummies, so every step issues the same number of DMAs.
      constexpr int NB2 = NB / 2;
      const int n_pairs = (n_tiles + 1) >> 1;
      auto issue2 = [&](int pp) {
        issue(2 * pp);
        if (2 * pp + 1 < n_tiles) {
          issue(2 * pp + 1);
        } else {
          const uint32_t slot = ring0 + (uint32_t)(((2 * pp + 1) % NB) * R::SLOT);
          issue_tile<D, BITS>(a, jl, slot, false, 0, lane, wv, rl64(bl.pg, 0), 0u, 0u, 0u);
        }
      };
#pragma unroll 1
      for (int pp = 0; pp < NB2 - 1 && pp < n_pairs; ++pp) issue2(pp);
      generic_tiles();
#pragma unroll 1
      for (int pp = 0; pp < n_pairs; ++pp) {
        const int ahead = (n_pairs - 1 - pp) < (NB2 - 2) ? (n_pairs - 1 - pp) : (NB2 - 2);
        wait_ahead<2 * R::M, NB2 - 2>(ahead);
        wg_barrier();
        if (pp + NB2 - 1 < n_pairs) issue2(pp + NB2 - 1);
        const int tt0 = 2 * pp, tt1 = tt0 + 1;
        const int b0 = tt0 >> tpb_shift, b1 = tt1 >> tpb_shift;
        if (sink.total > 0 && (pp & 1) == 0) range_priority(b_end - c0 - orig(b0) + sink.rem_after, sink.total);
        const bool ok0 = (m_blk >> b0) & 1, ok1 = tt1 < n_tiles && ((m_blk >> b1) & 1);
        const bool p0 = ok0 && piped(tt0), p1 = ok1 && piped(tt1);
        if (!live) continue;
        if (p0 && p1) {
          const int nv0 = seq_len - ((c0 + orig(b0)) << a.bs_shift) - ((tt0 & ((1 << tpb_shift) - 1)) << 4);
          const int nv1 = seq_len - ((c0 + orig(b1)) << a.bs_shift) - ((tt1 & ((1 << tpb_shift) - 1)) << 4);
          pair_step<D, QLO, BITS>(w, kc, ring + (tt0 % NB) * R::SLOT, ring + (tt1 % NB) * R::SLOT, nv0, nv1, lane);
        } else {
          if (p0) single(tt0);
          if (p1) single(tt1);
        }
      }
    } else {
      // Tile tt: wait for this wave's part of it, meet the others (every part has
      // landed; every wave is done with tile tt - 1), refill tt - 1's slot with
      // tile tt + NB - 1, compute tile tt.
#pragma unroll 1
      for (int tt = 0; tt < NB - 1 && tt < n_tiles; ++tt) issue(tt);
      generic_tiles();
#pragma unroll 1
      for (int tt = 0; tt < n_tiles; ++tt) {
        const int ahead = (n_tiles - 1 - tt) < (NB - 2) ? (n_tiles - 1 - tt) : (NB - 2);
        wait_tile<D, BITS, NB>(ahead);
        wg_barrier();
        if (tt + NB - 1 < n_tiles) issue(tt + NB - 1);
        const int b = tt >> tpb_shift;
        const int bo = orig(b);
        if (sink.total > 0 && (tt & 3) == 0) range_priority(b_end - c0 - bo + sink.rem_after, sink.total);
        if (!((m_blk >> b) & 1)) continue;
        if (!piped(tt)) continue;  // computed by generic_tiles
        if (!live && !pair) continue;
        single(tt);
      }
    }
    wait_vmcnt<0>();  // nothing of this chunk may still be landing in the ring
    wg_barrier();     // every wave is done reading the ring before the next chunk refills it
  }

  if (!carried) return;  // no block of this pass's tier: the row keeps the earlier passes' result
  const float l = rows_sum(w.l_lane);
  if constexpr (PS) {
    const float mterm = rows_sum(w.acc_ml);  // the column's V min term, every row of its group
#pragma unroll
    for (int j = 0; j < W::CPM; ++j) w.acc[j] += mterm;
  } else {
#pragma unroll
    for (int j = 0; j < W::CPM; ++j) w.acc[j] += w.acc_m;  // the V min term, the same for the lane's channels
  }
  if (mine) {
    const long qh = (long)kh * a.gqa + a.g0 + qcol;
    if (sink.direct) {  // lane (c, n): channels (4c + i) * CPM + j of query head qh (of its half)
      const float inv = 1.0f / l;
      const long o = q_row * a.o_s0 + qh * a.o_s1 + half * D;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v[W::CPM];
#pragma unroll
        for (int j = 0; j < W::CPM; ++j) v[j] = w.acc[j][i] * inv;
        st_n<W::CPM>(a.out, a.out_dtype, o + (4 * c + i) * W::CPM, v);
      }
      return;
    }
    const long row = sink.part_row0 + qh * sink.part_stride;
    float* dst = a.acc + row * RD + half * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < W::CPM; ++j) dst[(4 * c + i) * W::CPM + j] = w.acc[j][i];
    }
    if (c == 0 && half == 0) {  // the two halves hold the same (max, sum); PS: the group-0 column
      a.ml[row * 2] = w.m_run - (float)kk;
      a.ml[row * 2 + 1] = l;
    }
  }
}

// Workgroup g takes work item g of the batch's non-empty (split, head group)
// pairs in sequence order (head groups of a split adjacent, so they read the
// same token rows together). The grid is sized for every sequence at its
// maximum split count; workgroups past the last non-empty item exit at once,
// and they come last in dispatch order instead of between the busy ones.
// Three waves per SIMD (<= 168 VGPRs) where the ring leaves LDS for three
// workgroups per CU; INT8's larger ring and the float32-query variant get two.
// PAIR: head size 256 as half-heads (DecodeArgs::pair), D = 128.
template <int D, int BITS, bool QLO, bool PAIR, int PS>
__global__ __launch_bounds__(64 * kHeadsPerGroup, (BITS == 8 || QLO) ? 2 : 3) void decode_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring_lds[];
  SpanPass pass{false, true, 0, false};
  if (a.tier_mask) {  // a tier pass: nothing to do unless the layer holds this tier
    int m = *a.tier_mask & (2 | 4 | 8);
    if (m == 0) m = a.tier0;
    if (!(m & BITS)) return;
    const int lowest = m & -m;
    pass = SpanPass{true, BITS == lowest, m, BITS != lowest};
  }
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar job branches
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)ring_lds);
  const int n_hg = (a.L.H + kHeadsPerGroup - 1) / kHeadsPerGroup;
  // The head groups of one split read neighbouring bytes of the same rows, and
  // rows start 16 bytes into a 128-byte line (the page format's offsets), so
  // they share lines. Workgroups are dealt to the 8 XCDs round-robin by
  // dispatch order: put a split's head groups 8 dispatches apart (same XCD,
  // same L2) so a shared line is fetched from HBM once.
  const long span = 8L * n_hg;
  const long r = blockIdx.x % span;
  const long item = blockIdx.x - r + (r % 8) * n_hg + r / 8;
  const int incl0 = scan_chunk(a, 0, lane);
  if (a.num_seqs <= 64 && item >= (long)scan_total(incl0) * n_hg) return;  // past the last non-empty split
  long seq;
  int split;
  if (!locate(a, item / n_hg, lane, incl0, seq, split)) return;
  const int n_blocks = ((int)a.lens[seq] + a.L.BS - 1) >> a.bs_shift;
  const int bps = split_blocks(a, n_blocks);
  const int b_start = split * bps;
  const int b_end = b_start + bps < n_blocks ? b_start + bps : n_blocks;
  // INT2 splits take the range-share wave priorities too (cfg2 INT2 layer-step
  // 103.8 -> 100.1 us); INT4 measured the same with them and INT8 8.8 us slower.
  constexpr bool kPrio = BITS == 2;
  decode_span<D, BITS, QLO, true, PAIR, PS>(a, seq, b_start, b_end, (int)(item % n_hg), wv, lane, ring_lds, ring0,
                                  SpanSink{seq * a.hq * a.num_splits + split, a.num_splits, false, 0,
                                           kPrio ? b_end - b_start : 0}, pass);
}

// ---------------------------------------------------------------------------
// Balanced schedule. The batch's blocks, sequence after sequence, are cut into
// `ranges` contiguous ranges of equal cost (a live sequence costs its blocks plus
// kSeqCost for its span start-up; range r covers costs [r C / R, (r+1) C / R) of
// C in all): one persistent workgroup per range and head group, as many as the
// chip holds at once, so every workgroup streams about the same work and none
// waits for a late one. A sequence that lies inside one range
// is written straight to its output row; the pieces of a longer one (each
// range's first and last span) go to partial slots 2r and 2r + 1 and a merge
// kernel combines them. Ranges depend on the whole batch, so results are not
// batch-invariant (the split schedule is).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int seq_blocks(const DecodeArgs& a, long s) {
  const long len = s < a.num_seqs ? a.lens[s] : 0;
  return len > 0 ? (int)((len + a.L.BS - 1) >> a.bs_shift) : 0;
}

// A wave-uniform value held in a scalar register (the compiler cannot tell that a
// reduction's result is the same in every lane).
__device__ __forceinline__ long uni(long x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (long)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ long wave_total(long x) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

// The balanced partition weighs each live sequence as its blocks plus kSeqCost:
// a range that starts a sequence pays a span start-up (block facts, the ring's
// fill, the open K group's tile), about kSeqCost tiles of streaming, so ranges
// holding sequence boundaries get fewer blocks and end with the others. (cfg2
// INT4 layer-step: 6 -> 97.2 us, 0 -> 100.5 us; 4, 8, 10 and 12 measured no better.)
constexpr int kSeqCost = 6;
__device__ __forceinline__ int seq_cost(int nb) { return nb > 0 ? nb + kSeqCost : 0; }

// Total cost of the batch (every lane gets it).
__device__ __forceinline__ long batch_cost(const DecodeArgs& a, int lane) {
  long t = 0;
  for (long s0 = 0; s0 < a.num_seqs; s0 += 64) t += wave_total(seq_cost(seq_blocks(a, s0 + lane)));
  return t;
}

// floor(n / d) for 0 <= n < 2^53 and 0 < d < 2^31. n and d are exact in f64 and the
// f64 quotient is correctly rounded, so truncating it gives floor(n / d), or one
// more when rounding carried a quotient just under an integer up to it; one
// integer product takes that back. About 15 instructions against about 50 for a
// 64-bit integer division, on the start-up chain of every decode workgroup and
// merge wave.
__device__ __forceinline__ long div_floor(long n, long d) {
  long q = (long)((double)n / (double)d);
  if (q * d > n) --q;
  return q;
}

// First block of range r (of `ranges` over T blocks).
__device__ __forceinline__ long range_begin(long r, long ranges, long T) { return div_floor(r * T, ranges); }

// Range r's blocks [lo, hi) under the cost partition, and the sequence holding
// block lo with its first block: one walk over the lengths (64 sequences per step)
// places both ends.
__device__ __forceinline__ void range_blocks(const DecodeArgs& a, long r, int lane, long& seq, long& first, long& lo,
                                             long& hi) {
  const long CT = uni(batch_cost(a, lane));
  const long c0 = range_begin(r, a.ranges, CT), c1 = range_begin(r + 1, a.ranges, CT);
  long base_c = 0, base_b = 0;
  bool found = false;
  seq = a.num_seqs;
  for (long s0 = 0; s0 < a.num_seqs; s0 += 64) {
    const int nb = seq_blocks(a, s0 + lane);
    const int cost = seq_cost(nb);
    const int incl_c = wave_incl_scan(cost, lane), incl_b = wave_incl_scan(nb, lane);
    const int tot_c = __builtin_amdgcn_readlane(incl_c, 63);
    // The block at cost c in this step's sequences: lanes whose costs end at or
    // before c come before it.
    auto at = [&](long c, long& sq, long& f) -> long {
      const int k = __builtin_popcountll(__builtin_amdgcn_ballot_w64(base_c + incl_c <= c));
      sq = s0 + k;
      const long cum = base_c + __builtin_amdgcn_readlane(incl_c, k) - __builtin_amdgcn_readlane(cost, k);
      f = base_b + __builtin_amdgcn_readlane(incl_b, k) - __builtin_amdgcn_readlane(nb, k);
      const long off = c - cum - kSeqCost;
      return f + (off > 0 ? off : 0);
    };
    if (!found && c0 < base_c + tot_c) {
      lo = at(c0, seq, first);
      found = true;
    }
    if (c1 < base_c + tot_c) {
      long s2, f2;
      hi = at(c1, s2, f2);
      return;
    }
    base_c += tot_c;
    base_b += __builtin_amdgcn_readlane(incl_b, 63);
  }
  if (!found) {
    lo = base_b;
    first = base_b;
  }
  hi = base_b;
}

template <int D, int BITS, bool QLO, bool PAIR, int PS>
__global__ __launch_bounds__(64 * kHeadsPerGroup, (BITS == 8 || QLO) ? 2 : 3) void decode_balanced_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring_lds[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)ring_lds);
  const int n_hg = (a.L.H + kHeadsPerGroup - 1) / kHeadsPerGroup;
  // A range's head groups 8 dispatches apart: same XCD, shared L2 lines.
  const long span = 8L * n_hg;
  const long rr = blockIdx.x % span;
  const long item = blockIdx.x - rr + (rr % 8) * n_hg + rr / 8;
  const long r = item / n_hg;
  const int hg = (int)(item % n_hg);
  if (r >= a.ranges) return;
  long seq, first, lo, hi;
  range_blocks(a, r, lane, seq, first, lo, hi);
  lo = uni(lo);
  hi = uni(hi);
  if (lo >= hi) return;
  seq = uni(seq);
  first = uni(first);
  for (long pos = lo; pos < hi && seq < a.num_seqs;) {
    const int nb = (int)uni(seq_blocks(a, seq));
    const long end = first + nb < hi ? first + nb : hi;
    if (nb > 0) {
      const bool whole = pos == first && end == first + nb;
      const long slot = 2 * r + (pos == lo ? 0 : 1);
      decode_span<D, BITS, QLO, false, PAIR, PS>(a, seq, (int)(pos - first), (int)(end - first), hg, wv, lane, ring_lds,
                                       ring0, SpanSink{slot * a.hq, 1, whole, (int)(hi - end), (int)(hi - lo)});
    }
    pos = end;
    first += nb;
    ++seq;
  }
}

// Merge of a balanced decode: one wave per (sequence, query head) whose blocks
// span several ranges; the pieces sit in slot 2 rf + 1 (or 2 rf when the
// sequence starts its first range) and 2 r for the ranges after it. Lane i
// takes piece g + i's (max, sum) pair; the partial rows are then requested 16
// at a time, so a sequence's merge costs a few memory round trips rather than
// one per piece. A range left empty (fewer blocks than ranges) holds no piece:
// its weight is 0 and its slot is not read.
template <int D>
__global__ __launch_bounds__(256) void merge_balanced_kernel(DecodeArgs a) {
  constexpr int C = D / 64;
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);  // seq * hq + head
  if (row >= a.num_seqs * a.hq) return;
  const long seq = row / a.hq;
  const int head = (int)(row % a.hq);
  if (head % a.gqa < a.g0 || head % a.gqa >= a.g0 + a.gs) return;  // another pass's query heads
  const int nb = seq_blocks(a, seq);
  if (nb == 0) return;
  long cum = 0, CT;  // the sequence's first cost coordinate (its blocks start kSeqCost later); the batch's
  if (a.num_seqs <= 64) {  // one load of the lengths for both
    const int cl = seq_cost(seq_blocks(a, lane));
    cum = wave_total(lane < seq ? cl : 0);
    CT = wave_total(cl);
  } else {
    for (long s0 = 0; s0 < seq; s0 += 64) cum += wave_total(s0 + lane < seq ? seq_cost(seq_blocks(a, s0 + lane)) : 0);
    CT = batch_cost(a, lane);
  }
  cum = uni(cum);
  CT = uni(CT);
  const long R = a.ranges;
  // The range holding the block at cost c: range q covers costs [range_begin(q),
  // range_begin(q + 1)), and each block has a cost of its own. floor(c R / CT) is
  // that range or the one before it (range_begin rounds down: range q + 1 may start
  // at c itself), and empty ranges past it start at c too.
  auto range_of = [&](long c) {
    long q = div_floor(c * R, CT);
    while (range_begin(q + 1, R, CT) <= c) ++q;
    return q;
  };
  const long rf = range_of(cum + kSeqCost), rl = range_of(cum + kSeqCost + nb - 1);
  if (rf == rl) return;  // written directly by the decode kernel
  // The sequence is range rf's second span when the range starts at an earlier
  // sequence's cost (which maps to that sequence's blocks).
  const bool rf_second = range_begin(rf, R, CT) < cum;
  auto slot_of = [&](long q) { return 2 * q + (q == rf && rf_second ? 1 : 0); };
  const long n = rl - rf + 1;
  if (n <= 16) {
    // Up to 16 pieces: their (max, sum) pairs and partial rows are requested in
    // one round trip (which pieces exist follows from the ranges alone); the
    // weights are applied once the pairs are in.
    const int pi = lane & 15;
    const long qi = rf + pi;
    const bool mine = lane < 16 && pi < n && range_begin(qi, R, CT) < range_begin(qi + 1, R, CT);
    float mq = -__builtin_inff(), lq = 0.f;
    if (mine) {
      const long pr = slot_of(qi) * a.hq + head;
      mq = a.ml[pr * 2];
      lq = a.ml[pr * 2 + 1];
    }
    const uint64_t live = __builtin_amdgcn_ballot_w64(mine);  // piece u exists: bit u
    float x[16][C];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const long q = rf + u;
#pragma unroll
      for (int e = 0; e < C; ++e) x[u][e] = 0.f;
      if ((live >> u) & 1) {  // wave-uniform
        const float* src = a.acc + (slot_of(q) * a.hq + head) * D + C * lane;
#pragma unroll
        for (int e = 0; e < C; ++e) x[u][e] = src[e];
      }
    }
    float m = mq;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const float w = mine ? __builtin_amdgcn_exp2f(mq - m) : 0.f;
    float den = w * lq;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
    float o[C] = {};
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float wu = __shfl(w, u, 64);
#pragma unroll
      for (int e = 0; e < C; ++e) o[e] += x[u][e] * wu;
    }
#pragma unroll
    for (int e = 0; e < C; ++e) o[e] /= den;
    const long o_row = a.q_rows ? a.q_rows[seq] : seq;
    st_n<C>(a.out, a.out_dtype, o_row * a.o_s0 + head * a.o_s1 + C * lane, o);
    return;
  }
  float m = -__builtin_inff();
  for (long g = 0; g < n; g += 64) {
    const long q = rf + g + lane;
    if (q <= rl && range_begin(q, R, CT) < range_begin(q + 1, R, CT)) m = fmaxf(m, a.ml[(slot_of(q) * a.hq + head) * 2]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  float num[C] = {};
  float den = 0.f;
  for (long g = 0; g < n; g += 64) {
    const long q = rf + g + lane;
    float w = 0.f;
    if (q <= rl && range_begin(q, R, CT) < range_begin(q + 1, R, CT)) {
      const long pr = slot_of(q) * a.hq + head;
      w = __builtin_amdgcn_exp2f(a.ml[pr * 2] - m);
      den += a.ml[pr * 2 + 1] * w;
    }
    const int cnt = (int)(n - g < 64 ? n - g : 64);
    for (int u0 = 0; u0 < cnt; u0 += 16) {
      float x[16][C], wu[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        wu[u] = __shfl(w, (u0 + u) & 63, 64);  // piece g + u0 + u's weight (0 past the last)
        const float* src = a.acc + (slot_of(rf + g + u0 + u) * a.hq + head) * D + C * lane;
#pragma unroll
        for (int e = 0; e < C; ++e) x[u][e] = 0.f;
        if (u0 + u < cnt && wu[u] > 0.f) {
#pragma unroll
          for (int e = 0; e < C; ++e) x[u][e] = src[e];
        }
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
#pragma unroll
        for (int e = 0; e < C; ++e) num[e] += x[u][e] * wu[u];
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
  const long o_row = a.q_rows ? a.q_rows[seq] : seq;
  float o[C];
#pragma unroll
  for (int e = 0; e < C; ++e) o[e] = num[e] / den;
  st_n<C>(a.out, a.out_dtype, o_row * a.o_s0 + head * a.o_s1 + C * lane, o);
}

// Merge of the splits: one wave per (sequence, query head); lane l holds
// channels [D/64 * l, D/64 * (l + 1)). Up to 64 splits: the (max, sum) pairs
// and the first 16 splits' partial rows are requested together, so a row costs
// about one memory round trip; more splits take a slower two-pass loop.
template <int D>
__device__ __forceinline__ void merge_row(const MergeArgs& a, long row, long seq, int head, int used, int lane) {
  constexpr int C = D / 64;
  const long base = row * a.num_splits;
  float num[C] = {};
  float den = 0.f;
  if (used <= 64) {
    const float2 ml = lane < used ? ((const float2*)a.ml)[base + lane] : float2{-__builtin_inff(), 0.f};
    float w = 0.f;
    for (int g = 0; g < used; g += 16) {
      float x[16][C];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const long s = g + u < used ? g + u : 0;  // past the last split: split 0, unused
        const float* src = a.acc + (base + s) * D + C * lane;
        if constexpr (C == 4) {
          const float4 v = *(const float4*)src;
          x[u][0] = v.x;
          x[u][1] = v.y;
          x[u][2] = v.z;
          x[u][3] = v.w;
        } else if constexpr (C == 2) {
          const float2 v = *(const float2*)src;
          x[u][0] = v.x;
          x[u][1] = v.y;
        } else {
          x[u][0] = src[0];
        }
      }
      if (g == 0) {
        float m = ml.x;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        w = lane < used ? __builtin_amdgcn_exp2f(ml.x - m) : 0.f;
        den = ml.y * w;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (g + u < used) {
          const float ws = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(w), g + u));
#pragma unroll
          for (int e = 0; e < C; ++e) num[e] += x[u][e] * ws;
        }
      }
    }
  } else {
    float m = -__builtin_inff();
    for (int s0 = 0; s0 < used; s0 += 64) {
      const float mi = s0 + lane < used ? a.ml[(base + s0 + lane) * 2] : -__builtin_inff();
      m = fmaxf(m, mi);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    for (int s0 = 0; s0 < used; s0 += 64) {
      const bool in = s0 + lane < used;
      const float wl = in ? __builtin_amdgcn_exp2f(a.ml[(base + s0 + lane) * 2] - m) : 0.f;
      den += in ? a.ml[(base + s0 + lane) * 2 + 1] * wl : 0.f;
      const int cnt = used - s0 < 64 ? used - s0 : 64;
      for (int i = 0; i < cnt; ++i) {
        const float ws = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(wl), i));
        const float* src = a.acc + (base + s0 + i) * D + C * lane;
#pragma unroll
        for (int e = 0; e < C; ++e) num[e] += src[e] * ws;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
  }
  const long o_row = a.q_rows ? a.q_rows[seq] : seq;
  float o[C];
#pragma unroll
  for (int e = 0; e < C; ++e) o[e] = num[e] / den;
  st_n<C>(a.out, a.out_dtype, o_row * a.o_s0 + head * a.o_s1 + C * lane, o);
}

template <int D>
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);  // seq * hq + head
  if (row >= a.rows) return;
  const long seq = row / a.hq;
  const int head = (int)(row % a.hq);
  if (head % a.gqa < a.g0 || head % a.gqa >= a.g0 + a.gs) return;  // another pass's query heads
  const int seq_len = (int)a.lens[seq];
  if (seq_len <= 0) return;
  const int n_blocks = (seq_len + a.BS - 1) / a.BS;
  const int per = (n_blocks + a.num_splits - 1) / a.num_splits;
  const int bps = a.bps > per ? a.bps : per;
  const int used = (n_blocks + bps - 1) / bps;
  merge_row<D>(a, row, seq, head, used, lane);
}

// Dynamic LDS of a decode workgroup: the ring, and with PAIR the score exchange
// (every tier's ring leaves room for it at the workgroups per CU the launch bounds give).
template <int D, int BITS, bool PAIR, int PS>
constexpr int decode_lds() { return ring_slots<BITS, PS>() * Ring<D, BITS>::SLOT + (PAIR ? kPairLds : 0); }

template <int D, int BITS, bool QLO, bool PAIR, int PS>
hipError_t launch_decode_t(const DecodeArgs& a, hipStream_t s) {
  const dim3 block(64 * kHeadsPerGroup);
  constexpr int lds = decode_lds<D, BITS, PAIR, PS>();
  const long n_hg = (a.L.H + kHeadsPerGroup - 1) / kHeadsPerGroup;
  const long span = 8 * n_hg;  // the kernels permute workgroups within runs of `span`
  if (a.ranges > 0) {
    static std::atomic<uint64_t> attr_done{0};  // devices whose limit is raised, one bit each
    if (ensure_lds_limit((const void*)decode_balanced_kernel<D, BITS, QLO, PAIR, PS>, lds, &attr_done) != hipSuccess)
      return hipErrorInvalidValue;
    const long wgs = (a.ranges * n_hg + span - 1) / span * span;
    hipLaunchKernelGGL((decode_balanced_kernel<D, BITS, QLO, PAIR, PS>), dim3((unsigned)wgs), block, lds, s, a);
    return hipGetLastError();
  }
  static std::atomic<uint64_t> attr_done{0};
  if (ensure_lds_limit((const void*)decode_kernel<D, BITS, QLO, PAIR, PS>, lds, &attr_done) != hipSuccess)
    return hipErrorInvalidValue;
  const long items = (a.num_seqs * a.num_splits * n_hg + span - 1) / span * span;
  hipLaunchKernelGGL((decode_kernel<D, BITS, QLO, PAIR, PS>), dim3((unsigned)items), block, lds, s, a);
  return hipGetLastError();
}

// Workgroups of the balanced kernel the current device holds at once (cached per device).
template <int D, int BITS, bool QLO, bool PAIR, int PS>
hipError_t balanced_slots(long& slots) {
  constexpr int kMaxDevices = 64;
  static std::atomic<long> per_device[kMaxDevices];
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  long v = per_device[dev].load(std::memory_order_acquire);
  if (v <= 0) {
    int cus = 0, per_cu = 0;
    const size_t lds = (size_t)decode_lds<D, BITS, PAIR, PS>();
    static std::atomic<uint64_t> attr_done{0};
    if ((e = ensure_lds_limit((const void*)decode_balanced_kernel<D, BITS, QLO, PAIR, PS>, (int)lds, &attr_done)) !=
        hipSuccess)
      return e;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
             &per_cu, (const void*)decode_balanced_kernel<D, BITS, QLO, PAIR, PS>, 64 * kHeadsPerGroup, lds)) != hipSuccess)
      return e;
    v = (long)(cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
    per_device[dev].store(v, std::memory_order_release);
  }
  slots = v;
  return hipSuccess;
}

template <int D, bool QLO, bool PAIR, int PS>
hipError_t decode_slots_d(const DecodeArgs& a, long& slots) {
  if (a.tier == 8) return balanced_slots<D, 8, QLO, PAIR, PS>(slots);
  constexpr int PS1 = PS == 2 ? 1 : PS;  // as launch_decode_t4
  if (a.tier == 2) return balanced_slots<D, 2, QLO, PAIR, PS1>(slots);
  return balanced_slots<D, 4, QLO, PAIR, PS1>(slots);
}
template <int D, bool QLO, bool PAIR>
hipError_t decode_slots_p(const DecodeArgs& a, long& slots) {
  if constexpr (D == 128 && !PAIR)
    if (a.ps == 2) return decode_slots_d<D, QLO, PAIR, 2>(a, slots);
  return a.ps ? decode_slots_d<D, QLO, PAIR, 1>(a, slots) : decode_slots_d<D, QLO, PAIR, 0>(a, slots);
}

hipError_t decode_ranges(const DecodeArgs& a, long& ranges) {
  const bool qlo = a.q_dtype == ECHOKV_F32;
  long slots = 0;
  hipError_t e;
  if (a.L.D == 128 && a.pair)
    e = qlo ? decode_slots_p<128, true, true>(a, slots) : decode_slots_p<128, false, true>(a, slots);
  else if (a.L.D == 128)
    e = qlo ? decode_slots_p<128, true, false>(a, slots) : decode_slots_p<128, false, false>(a, slots);
  else if (a.L.D == 64 && !a.pair)
    e = qlo ? decode_slots_p<64, true, false>(a, slots) : decode_slots_p<64, false, false>(a, slots);
  else return hipErrorInvalidValue;
  if (e != hipSuccess) return e;
  const long n_hg = (a.L.H + kHeadsPerGroup - 1) / kHeadsPerGroup;
  long r = slots / n_hg;
  const long cap = a.num_seqs * a.num_splits / 2;  // two partial slots per range in the workspaces
  if (r > cap) r = cap;
  ranges = r > 0 ? r : 1;
  return hipSuccess;
}

// Two-tile steps (PS 2) run the INT8 kernel only: at INT2 / INT4 the step's
// operands do not fit the 168 registers that three waves per SIMD leave, and with
// two waves per SIMD those tiers decode slower than one tile at a time with three.
template <int D, bool QLO, bool PAIR, int PS>
hipError_t launch_decode_t4(const DecodeArgs& a, hipStream_t s) {
  if (a.tier == 8) return launch_decode_t<D, 8, QLO, PAIR, PS>(a, s);
  constexpr int PS1 = PS == 2 ? 1 : PS;
  if (a.tier == 2) return launch_decode_t<D, 2, QLO, PAIR, PS1>(a, s);
  return launch_decode_t<D, 4, QLO, PAIR, PS1>(a, s);
}
template <int D, bool QLO, bool PAIR>
hipError_t launch_decode_d(const DecodeArgs& a, hipStream_t s) {
  if constexpr (D == 128 && !PAIR)
    if (a.ps == 2) return launch_decode_t4<D, QLO, PAIR, 2>(a, s);
  return a.ps ? launch_decode_t4<D, QLO, PAIR, 1>(a, s) : launch_decode_t4<D, QLO, PAIR, 0>(a, s);
}

hipError_t launch_decode(const DecodeArgs& a, long num_seqs, hipStream_t s) {
  (void)num_seqs;  // a.num_seqs
  const bool qlo = a.q_dtype == ECHOKV_F32;
  if (a.L.D == 128 && a.pair) return qlo ? launch_decode_d<128, true, true>(a, s) : launch_decode_d<128, false, true>(a, s);
  if (a.pair) return hipErrorInvalidValue;
  if (a.L.D == 128) return qlo ? launch_decode_d<128, true, false>(a, s) : launch_decode_d<128, false, false>(a, s);
  if (a.L.D == 64) return qlo ? launch_decode_d<64, true, false>(a, s) : launch_decode_d<64, false, false>(a, s);
  return hipErrorInvalidValue;
}

hipError_t launch_merge_balanced(const DecodeArgs& a, hipStream_t s) {
  const long wgs = (a.num_seqs * a.hq + 3) / 4;
  const int d = a.pair ? 2 * a.L.D : a.L.D;  // the head size of the rows
  if (d == 128) hipLaunchKernelGGL(merge_balanced_kernel<128>, dim3((unsigned)wgs), dim3(256), 0, s, a);
  else if (d == 64) hipLaunchKernelGGL(merge_balanced_kernel<64>, dim3((unsigned)wgs), dim3(256), 0, s, a);
  else if (d == 256) hipLaunchKernelGGL(merge_balanced_kernel<256>, dim3((unsigned)wgs), dim3(256), 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// The workspaces (acc, ml) of echokv_decode_static: a file-scope device array.
// Each GPU the library runs on holds its own copy, at its own address, until the
// process ends. Host code never passes `scratch` itself to a kernel (in host code
// the name is a host-side stand-in, not a device address); it resolves the
// current device's address once with hipGetSymbolAddress and passes that.
static __device__ __align__(256) uint8_t scratch[kDecodeScratchBytes];

hipError_t decode_scratch(void** ptr) {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> per_device[kMaxDevices];  // zero-initialized: not resolved yet
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = per_device[dev].load(std::memory_order_acquire);
  if (!p) {  // first call on this device (a racing thread resolves the same address)
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    per_device[dev].store(p, std::memory_order_release);
  }
  *ptr = p;
  return hipSuccess;
}

hipError_t launch_merge(const MergeArgs& a, long num_seqs, hipStream_t s) {
  (void)num_seqs;
  const long wgs = (a.rows + 3) / 4;
  if (a.D == 128) hipLaunchKernelGGL(merge_kernel<128>, dim3((unsigned)wgs), dim3(256), 0, s, a);
  else if (a.D == 64) hipLaunchKernelGGL(merge_kernel<64>, dim3((unsigned)wgs), dim3(256), 0, s, a);
  else if (a.D == 256) hipLaunchKernelGGL(merge_kernel<256>, dim3((unsigned)wgs), dim3(256), 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace ek
