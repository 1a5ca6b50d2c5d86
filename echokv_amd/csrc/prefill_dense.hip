// Long-chunk prefill in two passes over a workspace of 64-key tiles
// (echokv_vllm/kernels/prefill.py:133-167, prefill_attention_dense: dequantize
// every context once, then one flash-attention call over the dense K/V).
//
// Pass 1, pack_kernel: one workgroup per (64-key tile of a request's context,
// KV head) dequantizes the keys once and writes the tile in the layout the
// attention pass reads:
//   K rows   [64 keys][D fp16 hi | D fp8 lo]    (lo = e4m3 of (x - hi) * 2^11: hi + lo
//                                                is the fp32 value to ~2^-15)
//   V^T rows [D][64 keys fp16]                  (keys of each 16-key step stored
//                                                in the MFMA operand order below)
// then padding to whole DMA rounds. Keys past the context and unreadable blocks
// are zeros.
//
// Pass 2, flash_kernel: one workgroup (8 waves) per (query tile, KV head). A
// query tile holds up to 256 / GQA tokens; its rows are (token, GQA head)
// pairs, 32 per wave. Workspace tiles stream through a three-slot LDS ring by
// LDS DMA (global_load_lds_dwordx4, 6 per wave per tile), the next tile in
// flight while the current one is consumed. Per wave and tile:
//   S^T[key, row] = K Q^T    v_mfma_f32_32x32x16_f16 on K hi (and Q lo for
//                            float32 queries), Q held in registers; K lo with
//                            Q as e4m3 on v_mfma_scale_f32_32x32x64_f8f6f4 (its
//                            scale operand takes the 2^11 back out) into the
//                            same accumulator: a quarter of the hi pass's cycles
//   online softmax per row   (the lane holds one row; its other half-wave holds
//                            the same row's other keys), max moved lazily
//   O^T[d, row] += V^T P^T   v_mfma_f32_32x32x16_f16, P^T straight from the S^T
//                            accumulator registers
// with the bottom-right causal limit key <= query position.
//
// LDS reads are conflict-free through XOR swizzles applied by the DMA address
// (the workspace itself stays linear): 16-byte slot s of K row k's hi part sits
// at slot s ^ (k & (D/8 - 1)) of that part, of its lo part at s ^ (k & (D/16 - 1)),
// slot s of V^T row d at s ^ ((d >> 1) & 7).
#include "args.h"

namespace ek {

namespace {

typedef float f16v_t __attribute__((ext_vector_type(16)));
typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef int v4i_t __attribute__((ext_vector_type(4)));

// K lo is stored as e4m3 of (x - hi) * 2^kLoShift; |x - hi| <= 2^-11 |x|, so the
// stored value stays within |x| (e4m3 holds up to 448; larger ones saturate).
constexpr int kLoShift = 11;
constexpr float kLoMax = 448.f;

constexpr int kDenseRing = 3;  // workspace tiles in the LDS ring

template <int D>
struct Ws {
  static constexpr int KHI = 2 * D;            // bytes of a key row's hi part (its lo part: D)
  static constexpr int KROW = 3 * D;           // bytes per key row (hi then lo)
  static constexpr int K_BYTES = kDenseKeys * KROW;
  static constexpr int VROW = 2 * kDenseKeys;  // bytes per V^T row
  static constexpr int V_BYTES = D * VROW;
  static constexpr int ROUND = 1024 * kDenseWaves;
  static constexpr int BYTES = (K_BYTES + V_BYTES + ROUND - 1) / ROUND * ROUND;  // = dense_tile_bytes(D)
  static constexpr int KSWH = D / 8 - 1;       // swizzle masks: 16-byte slots of the hi / lo part - 1
  static constexpr int KSWL = D / 16 - 1;
};

// Stored position of key k (0..63) in its V^T row: inside each 16-key step,
// bits 2 and 3 swap, so positions 8h..8h+7 hold keys {4h..4h+3, 8+4h..8+4h+3}
// -- the keys that half-wave h holds in rows 0..7 (or 8..15) of an S^T
// accumulator of v_mfma_f32_32x32x16 (lane l, register r: key 8(r/4) + 4(l/32) + r%4).
__device__ __forceinline__ int vpos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2" ::"v"(off), "s"(__builtin_amdgcn_readfirstlane(lds)),
               "s"(base)
               : "memory", "m0");
}

__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t u = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return (const uint8_t*)(((uint64_t)hi << 32) | lo);
}

// max / sum of x over the two half-waves (lanes l and l ^ 32).
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace

// ---- pass 1 ------------------------------------------------------------------

// One thread's CPT channels of one key at BITS: codes by vector loads (CPT * BITS / 8
// bytes, aligned to their size by the page format), K scale / min rows as fp16x8.
template <int BITS, int CPT>
struct Codes {
  static constexpr int BYTES = CPT * BITS / 8;
  static constexpr int WORDS = BYTES / 4;
  uint32_t w[WORDS];
  __device__ __forceinline__ void load(const uint8_t* p) {
    if constexpr (BYTES % 16 == 0) {
#pragma unroll
      for (int i = 0; i < BYTES / 16; ++i) {
        const uint4 v = ((const uint4*)p)[i];
        w[4 * i] = v.x, w[4 * i + 1] = v.y, w[4 * i + 2] = v.z, w[4 * i + 3] = v.w;
      }
    } else if constexpr (BYTES == 8) {
      const uint2 v = *(const uint2*)p;
      w[0] = v.x, w[1] = v.y;
    } else {
      w[0] = *(const uint32_t*)p;
    }
  }
  __device__ __forceinline__ float operator[](int e) const {
    return (float)((w[(e * BITS) / 32] >> ((e * BITS) % 32)) & ((1u << BITS) - 1u));
  }
};

template <int BITS, int D>
__device__ __forceinline__ void dequant_key(const PackArgs& a, long blk, int off, long rb, bool in_res, long rs,
                                            int h, int cq, float* kx, float* vx) {
  constexpr int CPT = D / 4;
  const Lay& L = a.L;
  const int c0 = cq * CPT;
  const long hb = (long)h * (D * BITS / 8) + c0 * BITS / 8;
  Codes<BITS, CPT> vc;
  vc.load(a.pages + rb + (long)L.H * D * BITS / 8 + hb);
  const int G = D / L.VG;
  const long pg = blk * L.stride;
  if (L.VG % CPT == 0) {  // the thread's channels share one (scale, min)
    const long ve = ((long)off * L.H + h) * G + c0 / L.VG;
    const float vs = (float)*f16p(a.pages, pg + L.o_vs + 2 * ve);
    const float vm = (float)*f16p(a.pages, pg + L.o_vm + 2 * ve);
#pragma unroll
    for (int e = 0; e < CPT; ++e) vx[e] = vc[e] * vs + vm;
  } else {
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const long ve = ((long)off * L.H + h) * G + (c0 + e) / L.VG;
      vx[e] = vc[e] * (float)*f16p(a.pages, pg + L.o_vs + 2 * ve) + (float)*f16p(a.pages, pg + L.o_vm + 2 * ve);
    }
  }
  if (in_res) {
#pragma unroll
    for (int q4 = 0; q4 < CPT / 4; ++q4)
      ld4(a.res.ptr, a.res.dtype, rs * a.res.s0 + (long)(off % L.KG) * a.res.s1 + h * a.res.s2 + c0 + 4 * q4,
          &kx[4 * q4]);
    return;
  }
  Codes<BITS, CPT> kc;
  kc.load(a.pages + rb + hb);
  const long se = ((long)(off / L.KG) * L.H + h) * D + c0;
  const h8_t* ks = (const h8_t*)(a.pages + pg + L.o_ks + 2 * se);
  const h8_t* km = (const h8_t*)(a.pages + pg + L.o_km + 2 * se);
#pragma unroll
  for (int v8 = 0; v8 < CPT / 8; ++v8) {
    const h8_t s8 = ks[v8], m8 = km[v8];
#pragma unroll
    for (int e = 0; e < 8; ++e) kx[8 * v8 + e] = kc[8 * v8 + e] * (float)s8[e] + (float)m8[e];
  }
}

template <int D>
__global__ __launch_bounds__(256) void pack_kernel(PackArgs a) {
  using W = Ws<D>;
  constexpr int CPT = D / 4;  // channels per thread: 4 threads per key
  __shared__ __attribute__((aligned(16))) _Float16 vt[D * kDenseKeys];
  const Lay& L = a.L;
  const int32_t* w = a.packs + blockIdx.x * 3;
  const long req = w[0];
  const int k0 = w[1], kv_end = w[2];
  const int h = blockIdx.y;
  const int tid = threadIdx.x, key = tid >> 2, cq = tid & 3;
  const int kp = k0 + key;
  float kx[CPT], vx[CPT];
#pragma unroll
  for (int e = 0; e < CPT; ++e) kx[e] = vx[e] = 0.f;
  if (kp < kv_end) {
    const long blk = a.bt[req * a.bt_s0 + kp / L.BS];
    const int off = kp % L.BS;
    if (blk >= 0 && blk < L.nb) {
      const int bits = tier_of(a.pages[blk * L.stride]);
      const long rb = row_base(a.pages, L, blk, off, bits);
      if (rb >= 0) {
        const long rs = a.block_res[blk];
        const bool in_res = rs >= 0 && rs < a.res.rows && a.res_group[rs] == off / L.KG;
        if (bits == 8) dequant_key<8, D>(a, blk, off, rb, in_res, rs, h, cq, kx, vx);
        else if (bits == 4) dequant_key<4, D>(a, blk, off, rb, in_res, rs, h, cq, kx, vx);
        else dequant_key<2, D>(a, blk, off, rb, in_res, rs, h, cq, kx, vx);
      }
    }
  }
  uint8_t* tile = a.ws + ((long)blockIdx.x * L.H + h) * W::BYTES;
  uint8_t* krow = tile + key * W::KROW;
#pragma unroll
  for (int v16 = 0; v16 < CPT / 16; ++v16) {
    h8_t hi[2];
    v4i_t lo;
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float x0 = kx[16 * v16 + e], x1 = kx[16 * v16 + e + 1];
      const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
      hi[e >> 3][e & 7] = h0;
      hi[e >> 3][(e & 7) + 1] = h1;
      const float l0 = fminf(fmaxf(__builtin_ldexpf(x0 - (float)h0, kLoShift), -kLoMax), kLoMax);
      const float l1 = fminf(fmaxf(__builtin_ldexpf(x1 - (float)h1, kLoShift), -kLoMax), kLoMax);
      const int pair = __builtin_amdgcn_cvt_pk_fp8_f32(l0, l1, 0, false) & 0xffff;
      if (e & 2) lo[e >> 2] |= pair << 16;
      else lo[e >> 2] = pair;
    }
    *(h8_t*)(krow + 2 * (cq * CPT + 16 * v16)) = hi[0];
    *(h8_t*)(krow + 2 * (cq * CPT + 16 * v16) + 16) = hi[1];
    *(v4i_t*)(krow + W::KHI + cq * CPT + 16 * v16) = lo;
  }
  const int vp = vpos(key);
#pragma unroll
  for (int e = 0; e < CPT; ++e) vt[(cq * CPT + e) * kDenseKeys + vp] = (_Float16)vx[e];
  __syncthreads();
  const uint4* src = (const uint4*)vt;
  uint4* dst = (uint4*)(tile + W::K_BYTES);
  for (int i = tid; i < W::V_BYTES / 16; i += 256) dst[i] = src[i];
}

// ---- pass 2 ------------------------------------------------------------------

template <int D, bool QLO, int NBUF>
__global__ __launch_bounds__(64 * kDenseWaves) void flash_kernel(FlashArgs a) {
  using W = Ws<D>;
  constexpr int NS = D / 16;   // 16-channel steps of S^T
  constexpr int NDB = D / 32;  // 32-channel blocks of O^T
  static_assert(NBUF == 2 || NBUF == 3, "two or three ring slots");
  constexpr int NDMA = W::BYTES / 1024 / kDenseWaves;
  static_assert(W::BYTES % (1024 * kDenseWaves) == 0, "tile must split into whole DMA rounds");
  constexpr int NLO = D / 64;   // 64-channel chunks of K lo
  constexpr int KGROUPS = NS / 2;          // K fragment groups per 64-key tile (= 2 * NLO)
  static_assert(2 * NDB <= 8, "V^T fragments of two steps fit one group");
  constexpr float kInf = __builtin_inff();
  extern __shared__ __attribute__((aligned(1024))) uint8_t ring[];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int j = lane & 31, hh = lane >> 5;

  // Items (query tile, head) are dealt to the 8 XCDs round-robin by dispatch
  // order; map dispatch b so that XCD b % 8 takes a contiguous run of items:
  // the query tiles of one request and head run on one XCD and share its L2.
  const long N = (long)a.n_qtiles * a.H;
  const long b = blockIdx.x;
  const long q8 = N / 8;
  const long item = b < 8 * q8 ? (b % 8) * q8 + b / 8 : b;
  const int h = (int)(item / a.n_qtiles);
  const int qt = (int)(item % a.n_qtiles);

  const int32_t* td = a.qtiles + qt * 5;
  const long q_row0 = td[0];
  const int n_tok = td[1], q_pos0 = td[2], ctx = td[3];
  const long t0 = td[4];
  const int gqa = a.gqa;
  const int n_rows = n_tok * gqa;
  const int kv_end = min(ctx, q_pos0 + n_tok);
  long nk = (kv_end + kDenseKeys - 1) / kDenseKeys;
  nk = t0 < 0 ? 0 : (nk < a.n_packs - t0 ? nk : a.n_packs - t0);  // never read past the workspace
  const int n_kt = nk > 0 ? (int)nk : 0;

  // This wave's rows and the keys they can see.
  const int r = 32 * wave + j;
  const bool rv = r < n_rows;
  const int last_r = min(32 * wave + 31, n_rows - 1);
  const bool active = 32 * wave < n_rows;
  const int qpos = q_pos0 + r / gqa;
  const int qmin = q_pos0 + (32 * wave) / gqa;
  const int qlim = og_limit(qpos, a.og_mask);                      // keys < qlim are visible
  const int qlim_min = a.og_mask ? (qmin & a.og_mask) : qmin + 1;  // at most the wave's smallest limit
  const int kend_w = active ? min(kv_end, q_pos0 + last_r / gqa + 1) : 0;  // keys this wave needs

  // DMA lane offsets inside a workspace tile (swizzled so that LDS reads are
  // conflict-free): wave w's i-th DMA fills LDS bytes [1024 (NDMA w + i), +1024).
  uint32_t doff[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int p = 1024 * (NDMA * wave + i) + 16 * lane;
    if (p < W::K_BYTES) {
      const int k = p / W::KROW, rb = p % W::KROW;
      doff[i] = rb < W::KHI ? k * W::KROW + 16 * ((rb / 16) ^ (k & W::KSWH))
                            : k * W::KROW + W::KHI + 16 * (((rb - W::KHI) / 16) ^ (k & W::KSWL));
    } else if (p < W::K_BYTES + W::V_BYTES) {
      const int q = p - W::K_BYTES;
      const int d = q / W::VROW, slot = (q % W::VROW) / 16;
      doff[i] = W::K_BYTES + d * W::VROW + 16 * (slot ^ ((d >> 1) & 7));
    } else {
      doff[i] = p;  // padding
    }
  }
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)ring);
  const uint8_t* gbase = a.ws + (t0 * a.H + h) * (long)W::BYTES;
  const long tstride = (long)a.H * W::BYTES;
  auto issue = [&](int kt) {
    const uint8_t* g = uniform_ptr(gbase + kt * tstride);
    const uint32_t m = ring0 + (uint32_t)((kt % NBUF) * W::BYTES + 1024 * NDMA * wave);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(g, doff[i], m + 1024 * i);
  };
#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i)
    if (i < n_kt) issue(i);

  // Query fragments (B operand of S^T): row r, channels 16 s + 8 hh .. +8 as fp16;
  // for K lo, channels 64 c + 32 hh .. +32 as e4m3.
  h8_t qf[NS], ql[QLO ? NS : 1];
  v8i_t qe[NLO];
  {
    const int tok = rv ? r / gqa : 0;
    const int qh = h * gqa + (rv ? r % gqa : 0);
    const long qb = (q_row0 + tok) * a.q_s0 + (long)qh * a.q_s1 + 8 * hh;
#pragma unroll
    for (int c = 0; c < NLO; ++c) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float x[8];
        if (rv) {
          ld_n<8>(a.q, a.q_dtype, qb - 8 * hh + 64 * c + 32 * hh + 8 * u, x);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = 0.f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = fminf(fmaxf(x[e], -kLoMax), kLoMax);
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const int lo2 = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * w], x[4 * w + 1], 0, false) & 0xffff;
          const int hi2 = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * w + 2], x[4 * w + 3], 0, false) & 0xffff;
          qe[c][2 * u + w] = lo2 | (hi2 << 16);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      float x[8];
      if (rv) {
        ld_n<8>(a.q, a.q_dtype, qb + 16 * s, x);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qf[s][e] = (_Float16)x[e];
        if constexpr (QLO) ql[s][e] = (_Float16)(x[e] - (float)qf[s][e]);
      }
    }
  }

  f16v_t acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f16v_t{};
  float m_run = -kInf, lsum = 0.f;
  const float sl2 = a.scale_log2;
  f16v_t s[2];
  h8_t fr[2][8];

  // S^T = K Q^T over two 32-key blocks. K fragments go in groups: hi of two
  // 16-channel steps for both blocks (4 x 16 bytes) and lo of 64-channel chunk
  // g / 2 for block g % 2 (32 bytes); the next group's LDS reads are in flight
  // while the current group feeds the MFMAs, which alternate between the two
  // blocks' accumulators (scheduling fences keep that order).
  auto kload = [&](const uint8_t* buf, int g, h8_t* dst) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int st = 2 * g + (i >> 1), kb = i & 1;
      const int k = 32 * kb + j;
      dst[i] = *(const h8_t*)(buf + k * W::KROW + 16 * ((2 * st + hh) ^ (k & W::KSWH)));
    }
    const int k = 32 * (g & 1) + j;
    const uint8_t* lr = buf + k * W::KROW + W::KHI;
    const int s0 = 4 * (g >> 1) + 2 * hh;
    dst[4] = *(const h8_t*)(lr + 16 * (s0 ^ (k & W::KSWL)));
    dst[5] = *(const h8_t*)(lr + 16 * ((s0 + 1) ^ (k & W::KSWL)));
  };
  auto qk = [&](const uint8_t* buf) {
    s[0] = f16v_t{};
    s[1] = f16v_t{};
    kload(buf, 0, fr[0]);
#pragma unroll
    for (int g = 0; g < KGROUPS; ++g) {
      if (g + 1 < KGROUPS) kload(buf, g + 1, fr[(g + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const h8_t* f = fr[g & 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int st = 2 * g + (i >> 1), kb = i & 1;
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i], qf[st], s[kb], 0, 0, 0);
      }
      {
        const v4i_t x0 = __builtin_bit_cast(v4i_t, f[4]), x1 = __builtin_bit_cast(v4i_t, f[5]);
        const v8i_t lo = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
        // e4m3 x e4m3; B's scale 2^(116 - 127) undoes the stored 2^11.
        s[g & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(lo, qe[g >> 1], s[g & 1], 0, 0, 0, 127, 0,
                                                                   127 - kLoShift);
      }
      if constexpr (QLO) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int st = 2 * g + (i >> 1), kb = i & 1;
          s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i], ql[st], s[kb], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // V^T fragments of keys 32 half .. 32 half + 31 (two 16-key steps).
  auto vload = [&](const uint8_t* buf, int half, h8_t* dst) {
#pragma unroll
    for (int i = 0; i < 2 * NDB; ++i) {
      const int ks = 2 * half + i / NDB, db = i % NDB;
      const int d = 32 * db + j;
      const int slot = (2 * ks + hh) ^ ((d >> 1) & 7);
      dst[i] = *(const h8_t*)(buf + W::K_BYTES + d * W::VROW + 16 * slot);
    }
  };
  // Online softmax of the tile at key kbase: S^T becomes P^T in place (the
  // first V^T fragments, issued before, are in flight meanwhile).
  auto softmax = [&](int kbase) {
    __builtin_amdgcn_sched_barrier(0);
    // Causal / context limit, only where this tile reaches it.
    if (kbase + kDenseKeys > qlim_min || kbase + kDenseKeys > kv_end) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kk = kbase + 32 * kb + 8 * (i >> 2) + 4 * hh + (i & 3);
          if (!(kk < kv_end && kk < qlim)) s[kb][i] = -kInf;
        }
      }
    }
    float mx = -kInf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
    }
    const float mt = halves_max(mx) * sl2;
    // Lazy rescale: the running max moves only when a row's tile max passes
    // it by more than 8 (log2 units); probabilities stay below 2^8 meanwhile.
    if (__builtin_amdgcn_ballot_w64(mt > m_run + 8.f)) {
      const float mn = fmaxf(m_run, mt);
      const float alpha = mn == -kInf ? 1.f : __builtin_amdgcn_exp2f(m_run - mn);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
      m_run = mn;
    }
    const float ms = m_run == -kInf ? 0.f : m_run;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kb][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], sl2, -ms));
    }
  };
  // O^T += V^T P^T, 16 keys per step; keys 32..63's fragments load while
  // keys 0..31 feed the MFMAs.
  auto pv = [&](const uint8_t* buf) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if (half == 0) vload(buf, 1, fr[1]);
      __builtin_amdgcn_sched_barrier(0);
      const h8_t* f = fr[half];
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const int ks = 2 * half + k2;
        const int kb = ks >> 1, r0 = 8 * (ks & 1);
        h8_t pb;
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[e] = (_Float16)s[kb][r0 + e];
        // The row sum takes the fp16 weights the PV product uses (two per dot).
        const h2_t one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int e = 0; e < 8; e += 2) lsum = __builtin_amdgcn_fdot2(h2_t{pb[e], pb[e + 1]}, one, lsum, false);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[k2 * NDB + db], pb, acc[db], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto finish = [&](const uint8_t* buf, int kbase) {
    vload(buf, 0, fr[0]);
    softmax(kbase);
    pv(buf);
  };

  // Tiles kt + 1 .. kt + NBUF - 1 are in flight while tile kt is consumed.
  for (int kt = 0; kt < n_kt; ++kt) {
    // Tile kt has landed once at most the DMAs of the tiles after it remain.
    if (NBUF == 3 && kt + 1 < n_kt) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NDMA) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kt + NBUF - 1 < n_kt) issue(kt + NBUF - 1);
    const int kbase = kt * kDenseKeys;
    if (!active || kbase >= kend_w) continue;
    const uint8_t* buf = ring + (kt % NBUF) * W::BYTES;
    qk(buf);
    finish(buf, kbase);
  }

  const float l = halves_sum(lsum);
  if (!rv) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const long ob = (q_row0 + r / gqa) * a.o_s0 + (long)(h * gqa + r % gqa) * a.o_s1;
  if (a.lse && hh == 0) a.lse[(q_row0 + r / gqa) * a.hq + h * gqa + r % gqa] = l > 0.f ? m_run + __log2f(l) : -kInf;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = acc[db][4 * g + e] * inv;
      st_n<4>(a.out, a.out_dtype, ob + 32 * db + 8 * g + 4 * hh, o);
    }
  }
}

// ---- launchers ---------------------------------------------------------------

hipError_t launch_prefill_pack(const PackArgs& a, long n_packs, hipStream_t s) {
  const dim3 grid((unsigned)n_packs, (unsigned)a.L.H);
  if (a.L.D == 128) hipLaunchKernelGGL(pack_kernel<128>, grid, dim3(256), 0, s, a);
  else if (a.L.D == 64) hipLaunchKernelGGL(pack_kernel<64>, grid, dim3(256), 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int D, bool QLO>
static hipError_t flash_one(const FlashArgs& a, hipStream_t s) {
  constexpr int NBUF = kDenseRing;
  constexpr int lds = NBUF * Ws<D>::BYTES;
  static std::atomic<uint64_t> attr_done{0};  // devices whose limit is raised, one bit each
  const hipError_t e = ensure_lds_limit((const void*)flash_kernel<D, QLO, NBUF>, lds, &attr_done);
  if (e != hipSuccess) return e;
  const long n = (long)a.n_qtiles * a.H;
  hipLaunchKernelGGL((flash_kernel<D, QLO, NBUF>), dim3((unsigned)n), dim3(64 * kDenseWaves), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_prefill_flash(const FlashArgs& a, hipStream_t s) {
  const bool qlo = a.q_dtype == ECHOKV_F32;
  if (a.D == 128) return qlo ? flash_one<128, true>(a, s) : flash_one<128, false>(a, s);
  if (a.D == 64) return qlo ? flash_one<64, true>(a, s) : flash_one<64, false>(a, s);
  return hipErrorInvalidValue;
}

}  // namespace ek
