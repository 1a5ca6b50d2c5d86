// Device-side helpers shared by the EchoKV gfx950 kernels: page layout and
// addressing, storage numerics, element loads, small vector types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "echokv.h"

namespace ek {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// Layout as a by-value kernel argument.
struct Lay {
  int H, D, BS, KG, VG, KC;
  long nb, stride, o_vs, o_vm, o_ks, o_km, o_data, cb;
};

struct Res {
  void* ptr;
  int dtype, rows;
  long s0, s1, s2;
};

constexpr float kFp16Tiny = 6.103515625e-05f;  // 2^-14, smallest normal fp16

// ---- element loads / stores by dtype code --------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40);  // NaN stays NaN
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float ld(const void* p, int dtype, long i) {
  if (dtype == ECHOKV_F32) return ((const float*)p)[i];
  if (dtype == ECHOKV_F16) return (float)((const _Float16*)p)[i];
  return bf16_to_f32(((const uint16_t*)p)[i]);
}

__device__ __forceinline__ void st(void* p, int dtype, long i, float v) {
  if (dtype == ECHOKV_F32) ((float*)p)[i] = v;
  else if (dtype == ECHOKV_F16) ((_Float16*)p)[i] = (_Float16)v;
  else ((uint16_t*)p)[i] = f32_to_bf16(v);
}

// N consecutive elements starting at element i. The dtype branch sits outside
// the element loop, so the N loads issue back to back and the wave waits once
// (a branch per element would wait for each load before issuing the next).
template <int N>
__device__ __forceinline__ void ld_n(const void* p, int dtype, long i, float* x) {
  if (dtype == ECHOKV_F16) {
    const _Float16* s = (const _Float16*)p + i;
#pragma unroll
    for (int e = 0; e < N; ++e) x[e] = (float)s[e];
  } else if (dtype == ECHOKV_BF16) {
    const uint16_t* s = (const uint16_t*)p + i;
#pragma unroll
    for (int e = 0; e < N; ++e) x[e] = bf16_to_f32(s[e]);
  } else {
    const float* s = (const float*)p + i;
#pragma unroll
    for (int e = 0; e < N; ++e) x[e] = s[e];
  }
}

// Four consecutive elements (channels) starting at element i.
__device__ __forceinline__ void ld4(const void* p, int dtype, long i, float x[4]) { ld_n<4>(p, dtype, i, x); }

// N consecutive elements stored from x at element i (dtype branch outside the loop).
template <int N>
__device__ __forceinline__ void st_n(void* p, int dtype, long i, const float* x) {
  if (dtype == ECHOKV_F16) {
    _Float16* d = (_Float16*)p + i;
#pragma unroll
    for (int e = 0; e < N; ++e) d[e] = (_Float16)x[e];
  } else if (dtype == ECHOKV_BF16) {
    uint16_t* d = (uint16_t*)p + i;
#pragma unroll
    for (int e = 0; e < N; ++e) d[e] = f32_to_bf16(x[e]);
  } else {
    float* d = (float*)p + i;
#pragma unroll
    for (int e = 0; e < N; ++e) d[e] = x[e];
  }
}

// ---- tiers and addressing ------------------------------------------------
// A block's tier from its header tag: 4 and 8 as stored; 0 (never opened)
// and anything else are addressed as INT2, which stays inside the own page.
__device__ __forceinline__ int tier_of(uint32_t tag) { return (tag == 4u || tag == 8u) ? (int)tag : 2; }

// Byte offset (from the pages base) of the first byte of the chunk holding
// token `off` of block `blk` at `bits`, or -1 when the block's chunk table
// names a chunk outside this layer's pages.
__device__ __forceinline__ long chunk_base(const uint8_t* pages, const Lay& L, long blk, int off, int bits) {
  const int tpc = 2 * L.BS / bits;
  const int j = off / tpc;
  if (j == 0) return blk * L.stride + L.o_data;
  const int id = *(const int32_t*)(pages + blk * L.stride + 4 + 4 * (j - 1));
  const long page = id / L.KC, slot = id % L.KC;
  if (id < 0 || page >= L.nb) return -1;
  return page * L.stride + L.o_data + slot * L.cb;
}

// Byte offset of token `off`'s K+V row in block `blk` at `bits` (-1: bad chunk id).
__device__ __forceinline__ long row_base(const uint8_t* pages, const Lay& L, long blk, int off, int bits) {
  const long cb = chunk_base(pages, L, blk, off, bits);
  if (cb < 0) return -1;
  const int tpc = 2 * L.BS / bits;
  return cb + (long)(off % tpc) * (2L * L.H * L.D * bits / 8);
}

// A block's 16 header bytes, read once: [0] tag, [4:16] pool chunk ids.
struct Hdr {
  uint32_t tag;
  int32_t id0, id1, id2;  // pool chunk ids of chunks 1..3 (fields, not an array: no stack copy)
  // Chunk j's id (j in 0..2) by masks: a select chain over the fields lets the
  // compiler turn the header into a stack array indexed at run time.
  __device__ __forceinline__ int32_t id(int j) const {
    const int32_t m0 = -(int32_t)(j == 0), m1 = -(int32_t)(j == 1), m2 = -(int32_t)(j >= 2);
    return (id0 & m0) | (id1 & m1) | (id2 & m2);
  }
};

__device__ __forceinline__ Hdr load_hdr(const uint8_t* pages, const Lay& L, long blk) {
  const uint4 h = *(const uint4*)(pages + blk * L.stride);
  return Hdr{h.x & 0xffu, (int32_t)h.y, (int32_t)h.z, (int32_t)h.w};
}

// row_base from a header already in registers.
__device__ __forceinline__ long row_base_h(const Lay& L, long blk, const Hdr& hd, int off, int bits) {
  const int tpc = 2 * L.BS / bits;
  const int j = off / tpc;
  long cb = blk * L.stride + L.o_data;
  if (j > 0) {
    const int id = hd.id(j - 1);
    const long page = id / L.KC, slot = id % L.KC;
    if (id < 0 || page >= L.nb) return -1;
    cb = page * L.stride + L.o_data + slot * L.cb;
  }
  return cb + (long)(off % tpc) * (2L * L.H * L.D * bits / 8);
}

// ---- storage numerics (echokv_vllm/quant.py:26-75) ------------------------
// fp16-rounded (scale, min) of a group with float32 extremes mn, mx. Division
// is IEEE (correctly rounded), casts are round-to-nearest-even.
__device__ __forceinline__ void group_stats(float mn, float mx, int bits, _Float16& s16, _Float16& m16, float& s,
                                            float& m) {
#pragma clang fp contract(off)
  m16 = (_Float16)mn;
  m = (float)m16;
  const float levels = (float)((1 << bits) - 1);
  const float sc = fmaxf((mx - m) / levels, kFp16Tiny);
  s16 = (_Float16)sc;
  s = (float)s16;
}

__device__ __forceinline__ uint32_t quant_code(float x, float m, float s, int bits) {
#pragma clang fp contract(off)
  const float levels = (float)((1 << bits) - 1);
  float q = __builtin_rintf((x - m) / s);
  q = fminf(fmaxf(q, 0.0f), levels);
  return (uint32_t)q;
}

// Pack four codes (channels 4c..4c+3) little-endian inside bytes.
__device__ __forceinline__ uint32_t pack4(const uint32_t q[4], int bits) {
  return q[0] | (q[1] << bits) | (q[2] << (2 * bits)) | (q[3] << (3 * bits));
}

// Store the packed codes of four channels at byte address p (bits/2 bytes).
__device__ __forceinline__ void store_codes4(uint8_t* p, uint32_t packed, int bits) {
  if (bits == 8) *(uint32_t*)p = packed;
  else if (bits == 4) *(uint16_t*)p = (uint16_t)packed;
  else *p = (uint8_t)packed;
}

__device__ __forceinline__ uint32_t load_codes4(const uint8_t* p, int bits) {
  if (bits == 8) return *(const uint32_t*)p;
  if (bits == 4) return *(const uint16_t*)p;
  return *p;
}

__device__ __forceinline__ float code_at(uint32_t packed, int e, int bits) {
  return (float)((packed >> (e * bits)) & ((1u << bits) - 1u));
}

// Min / max over an aligned segment of `width` lanes (a power of two <= 64).
__device__ __forceinline__ void seg_minmax(float& mn, float& mx, int width) {
  for (int m = width >> 1; m > 0; m >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, m, 64));
    mx = fmaxf(mx, __shfl_xor(mx, m, 64));
  }
}

__device__ __forceinline__ _Float16* f16p(uint8_t* pages, long byte) { return (_Float16*)(pages + byte); }
__device__ __forceinline__ const _Float16* f16p(const uint8_t* pages, long byte) {
  return (const _Float16*)(pages + byte);
}

}  // namespace ek
