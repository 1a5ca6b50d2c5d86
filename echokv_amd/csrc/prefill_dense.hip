// Long-chunk prefill in two passes over a workspace of 64-key tiles
// (echokv_vllm/kernels/prefill.py:133-167, prefill_attention_dense: dequantize
// every context once, then one flash-attention call over the dense K/V).
//
// Pass 1, pack_kernel: one workgroup per (64-key tile of a request's context,
// KV head) dequantizes the keys once and writes the tile in the layout the
// attention pass reads:
//   K rows   [64 keys][D fp16 hi | D fp16 lo]   (hi + lo = the fp32 value to ~2^-22)
//   V^T rows [D][64 keys fp16]                  (keys of each 16-key step stored
//                                                in the MFMA operand order below)
// Keys past the context and unreadable blocks are zeros.
//
// Pass 2, flash_kernel: one workgroup (8 waves) per (query tile, KV head). A
// query tile holds up to 256 / GQA tokens; its rows are (token, GQA head)
// pairs, 32 per wave. Workspace tiles stream through a two-slot LDS ring by
// LDS DMA (global_load_lds_dwordx4, 6 per wave per tile), the next tile in
// flight while the current one is consumed. Per wave and tile:
//   S^T[key, row] = K Q^T    v_mfma_f32_32x32x16_f16 on K hi and K lo (and Q lo
//                            for float32 queries), Q held in registers
//   online softmax per row   (the lane holds one row; its other half-wave holds
//                            the same row's other keys), max moved lazily
//   O^T[d, row] += V^T P^T   v_mfma_f32_32x32x16_f16, P^T straight from the S^T
//                            accumulator registers
// with the bottom-right causal limit key <= query position.
//
// LDS reads are conflict-free through XOR swizzles applied by the DMA address
// (the workspace itself stays linear): 16-byte slot s of K row k sits at slot
// s ^ (k & 15) of its half-row, slot s of V^T row d at s ^ ((d >> 1) & 7).
#include "args.h"

namespace ek {

namespace {

typedef float f16v_t __attribute__((ext_vector_type(16)));

template <int D>
struct Ws {
  static constexpr int KROW = 4 * D;          // bytes per key row (hi then lo)
  static constexpr int K_BYTES = kDenseKeys * KROW;
  static constexpr int VROW = 2 * kDenseKeys;  // bytes per V^T row
  static constexpr int V_BYTES = D * VROW;
  static constexpr int BYTES = K_BYTES + V_BYTES;
  static constexpr int KSW = D / 8 - 1;       // K swizzle mask (16-byte slots per half-row - 1)
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
        const int grp = off / L.KG;
        const bool in_res = rs >= 0 && rs < a.res.rows && a.res_group[rs] == grp;
        const int G = D / L.VG;
        const long hb = (long)h * (D * bits / 8);
#pragma unroll
        for (int q4 = 0; q4 < CPT / 4; ++q4) {
          const int ch = cq * CPT + 4 * q4;
          const uint32_t vc = load_codes4(a.pages + rb + (long)L.H * D * bits / 8 + hb + ch * bits / 8, bits);
          const long ve = ((long)off * L.H + h) * G + ch / L.VG;
          const float vs = (float)*f16p(a.pages, blk * L.stride + L.o_vs + 2 * ve);
          const float vm = (float)*f16p(a.pages, blk * L.stride + L.o_vm + 2 * ve);
#pragma unroll
          for (int e = 0; e < 4; ++e) vx[4 * q4 + e] = code_at(vc, e, bits) * vs + vm;
          if (in_res) {
            ld4(a.res.ptr, a.res.dtype, rs * a.res.s0 + (long)(off % L.KG) * a.res.s1 + h * a.res.s2 + ch,
                &kx[4 * q4]);
          } else {
            const uint32_t kc = load_codes4(a.pages + rb + hb + ch * bits / 8, bits);
            const long se = ((long)grp * L.H + h) * D + ch;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float ks = (float)*f16p(a.pages, blk * L.stride + L.o_ks + 2 * (se + e));
              const float km = (float)*f16p(a.pages, blk * L.stride + L.o_km + 2 * (se + e));
              kx[4 * q4 + e] = code_at(kc, e, bits) * ks + km;
            }
          }
        }
      }
    }
  }
  uint8_t* tile = a.ws + ((long)blockIdx.x * L.H + h) * W::BYTES;
  uint8_t* krow = tile + key * W::KROW + 2 * cq * CPT;
#pragma unroll
  for (int v8 = 0; v8 < CPT / 8; ++v8) {
    h8_t hi, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = kx[8 * v8 + e];
      hi[e] = (_Float16)x;
      lo[e] = (_Float16)(x - (float)hi[e]);
    }
    *(h8_t*)(krow + 16 * v8) = hi;
    *(h8_t*)(krow + 2 * D + 16 * v8) = lo;
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

template <int D, bool QLO>
__global__ __launch_bounds__(64 * kDenseWaves) void flash_kernel(FlashArgs a) {
  using W = Ws<D>;
  constexpr int NS = D / 16;   // 16-channel steps of S^T
  constexpr int NDB = D / 32;  // 32-channel blocks of O^T
  constexpr int NDMA = W::BYTES / 1024 / kDenseWaves;
  static_assert(W::BYTES % (1024 * kDenseWaves) == 0, "tile must split into whole DMA rounds");
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
  const int kend_w = active ? min(kv_end, q_pos0 + last_r / gqa + 1) : 0;  // keys this wave needs

  // DMA lane offsets inside a workspace tile (swizzled so that LDS reads are
  // conflict-free): wave w's i-th DMA fills LDS bytes [1024 (NDMA w + i), +1024).
  uint32_t doff[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int p = 1024 * (NDMA * wave + i) + 16 * lane;
    if (p < W::K_BYTES) {
      const int k = p / W::KROW, rb = p % W::KROW;
      const int half = rb / (2 * D), slot = (rb % (2 * D)) / 16;
      doff[i] = k * W::KROW + half * 2 * D + 16 * (slot ^ (k & W::KSW));
    } else {
      const int q = p - W::K_BYTES;
      const int d = q / W::VROW, slot = (q % W::VROW) / 16;
      doff[i] = W::K_BYTES + d * W::VROW + 16 * (slot ^ ((d >> 1) & 7));
    }
  }
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)ring);
  const uint8_t* gbase = a.ws + (t0 * a.H + h) * (long)W::BYTES;
  const long tstride = (long)a.H * W::BYTES;
  auto issue = [&](int kt) {
    const uint8_t* g = uniform_ptr(gbase + kt * tstride);
    const uint32_t m = ring0 + (uint32_t)((kt & 1) * W::BYTES + 1024 * NDMA * wave);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(g, doff[i], m + 1024 * i);
  };
  if (n_kt > 0) issue(0);

  // Query fragments (B operand of S^T): row r, channels 16 s + 8 hh .. +8.
  h8_t qf[NS], ql[QLO ? NS : 1];
  {
    const int tok = rv ? r / gqa : 0;
    const int qh = h * gqa + (rv ? r % gqa : 0);
    const long qb = (q_row0 + tok) * a.q_s0 + (long)qh * a.q_s1 + 8 * hh;
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

  for (int kt = 0; kt < n_kt; ++kt) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kt + 1 < n_kt) issue(kt + 1);
    const int kbase = kt * kDenseKeys;
    if (!active || kbase >= kend_w) continue;
    const uint8_t* buf = ring + (kt & 1) * W::BYTES;

    // S^T = K Q^T over two 32-key blocks.
    f16v_t s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int k = 32 * kb + j;
      const uint8_t* kr = buf + k * W::KROW;
      s[kb] = f16v_t{};
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const int slot = (2 * st + hh) ^ (k & W::KSW);
        const h8_t khi = *(const h8_t*)(kr + 16 * slot);
        const h8_t klo = *(const h8_t*)(kr + 2 * D + 16 * slot);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(khi, qf[st], s[kb], 0, 0, 0);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(klo, qf[st], s[kb], 0, 0, 0);
        if constexpr (QLO) s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(khi, ql[st], s[kb], 0, 0, 0);
      }
    }

    // Causal / context limit, only where this tile reaches it.
    if (kbase + kDenseKeys > qmin + 1 || kbase + kDenseKeys > kv_end) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kk = kbase + 32 * kb + 8 * (i >> 2) + 4 * hh + (i & 3);
          if (!(kk < kv_end && kk <= qpos)) s[kb][i] = -kInf;
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
      for (int i = 0; i < 16; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], sl2, -ms));
        s[kb][i] = p;
        lsum += p;
      }
    }

    // O^T += V^T P^T, 16 keys per step.
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kb = ks >> 1, r0 = 8 * (ks & 1);
      h8_t pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = (_Float16)s[kb][r0 + e];
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int d = 32 * db + j;
        const int slot = (2 * ks + hh) ^ ((d >> 1) & 7);
        const h8_t va = *(const h8_t*)(buf + W::K_BYTES + d * W::VROW + 16 * slot);
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, acc[db], 0, 0, 0);
      }
    }
  }

  const float l = halves_sum(lsum);
  if (!rv) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const long ob = (q_row0 + r / gqa) * a.o_s0 + (long)(h * gqa + r % gqa) * a.o_s1;
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
  constexpr int lds = 2 * Ws<D>::BYTES;
  static bool attr = false;
  if (!attr) {
    const hipError_t e =
        hipFuncSetAttribute((const void*)flash_kernel<D, QLO>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    attr = true;
  }
  const long n = (long)a.n_qtiles * a.H;
  hipLaunchKernelGGL((flash_kernel<D, QLO>), dim3((unsigned)n), dim3(64 * kDenseWaves), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_prefill_flash(const FlashArgs& a, hipStream_t s) {
  const bool qlo = a.q_dtype == ECHOKV_F32;
  if (a.D == 128) return qlo ? flash_one<128, true>(a, s) : flash_one<128, false>(a, s);
  if (a.D == 64) return qlo ? flash_one<64, true>(a, s) : flash_one<64, false>(a, s);
  return hipErrorInvalidValue;
}

}  // namespace ek
