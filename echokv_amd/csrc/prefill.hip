// Chunked-prefill attention over the tiered pages on gfx950 MFMA tiles.
//
// One workgroup (4 waves) per (query tile, KV head). A tile holds up to
// 128 / GQA query tokens; its rows are (token, GQA head) pairs, 128 rows, 32
// per wave (two 16-row blocks) -- at head size 256, 64 / GQA tokens and one
// 16-row block per wave (RB), so a wave's accumulators and query fragments take
// the registers they take at 128. The context is walked in 32-key tiles: the
// workgroup dequantizes each key tile once into LDS -- K row-major as an fp16
// hi + lo pair (exact to ~2^-22), V transposed in fp16 -- and every wave then
// runs, per 16-row block,
//   S^T[key, row] = K Q^T         (v_mfma_f32_16x16x32_f16 on K hi and K lo)
//   O^T[d, row]  += V^T P^T       (v_mfma_f32_16x16x32_f16, D/16 per block)
// with a per-row online softmax and the bottom-right causal limit
// key <= query position (echokv_vllm/kernels/prefill.py:210-236 semantics).
// The S^T accumulator (lane = 4 keys x 1 row) is the P^T B-operand as is: the
// 32-key contraction maps lane group c's eight k-slots to keys
// {4c..4c+3, 16+4c..16+4c+3}, and the V^T A-operand reads the same keys.
#include "args.h"

namespace ek {

namespace {
constexpr int kKeys = 32;           // keys per LDS tile
constexpr int kKPad = 8;            // fp16 padding per K row
constexpr int kVPad = 8;            // fp16 padding per V^T row

__device__ __forceinline__ h2_t u2h_(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
}  // namespace

template <int D, bool QLO, int RB>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillArgs a) {
  constexpr int KS = D + kKPad;       // K tile row stride (halves)
  constexpr int VS = kKeys + kVPad;   // V^T row stride (halves)
  constexpr int NQK = D / 32;
  constexpr int NPV = D / 16;
  __shared__ __attribute__((aligned(16))) _Float16 kt[kKeys * KS];   // K, fp16 hi part
  __shared__ __attribute__((aligned(16))) _Float16 ktl[kKeys * KS];  // K, fp16 lo part
  __shared__ __attribute__((aligned(16))) _Float16 vt[D * VS];

  const Lay& L = a.L;
  const int tile = blockIdx.x;
  const int h = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane >> 4, n = lane & 15;
  const int32_t* td = a.tiles + tile * 5;
  const long q_row0 = td[0];
  const int n_tok = td[1], q_pos0 = td[2], ctx = td[3];
  const long req = td[4];
  const int gqa = a.gqa;
  const int n_rows = n_tok * gqa;

  // Query fragments (B operand of S^T): row = 16*RB*wave + 16*rb + n, channels
  // 32j + 8c .. +8 in natural order.
  h8_t qf[RB][NQK], qfl[RB][QLO ? NQK : 1];
  int qpos[RB], qlim[RB];  // keys < qlim are visible
  bool rvalid[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = 16 * RB * wave + 16 * rb + n;
    rvalid[rb] = r < n_rows;
    const int tok = rvalid[rb] ? r / gqa : 0;
    const int hh = h * gqa + (rvalid[rb] ? r % gqa : 0);
    qpos[rb] = q_pos0 + tok;
    qlim[rb] = og_limit(qpos[rb], a.og_mask);
    const long qb = (q_row0 + tok) * a.q_s0 + (long)hh * a.q_s1;
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = rvalid[rb] ? ld(a.q, a.q_dtype, qb + 32 * j + 8 * c + e) : 0.f;
        qf[rb][j][e] = (_Float16)x;
        if constexpr (QLO) qfl[rb][j][e] = (_Float16)(x - (float)qf[rb][j][e]);
      }
    }
  }
  f4_t acc[RB][NPV];
  float m_run[RB], l_lane[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int j = 0; j < NPV; ++j) acc[rb][j] = f4_t{0.f, 0.f, 0.f, 0.f};
    m_run[rb] = -__builtin_inff();
    l_lane[rb] = 0.f;
  }

  int kv_end = q_pos0 + n_tok;
  kv_end = kv_end < ctx ? kv_end : ctx;
  // Dequantization mapping: thread -> (key t, 8 channels block cb).
  constexpr int CPT = D / 8;  // channels per thread (8 threads per key)
  const int dt = tid >> 3, dcb = tid & 7;
  for (int k0 = 0; k0 < kv_end; k0 += kKeys) {
    __syncthreads();
    {
      const int kp = k0 + dt;
      float kx[CPT], vx[CPT];
#pragma unroll
      for (int e = 0; e < CPT; ++e) kx[e] = vx[e] = 0.f;
      if (kp < kv_end) {
        const long blk = a.bt[req * a.bt_s0 + kp / L.BS];
        const int off = kp % L.BS;
        if (blk >= 0 && blk < L.nb) {
          const int bits = tier_of(a.pages[blk * L.stride]);
          const long rb = row_base(a.pages, L, blk, off, bits);
          const long rs = a.block_res[blk];
          const int grp = off / L.KG;
          const bool in_res = rs >= 0 && rs < a.res.rows && a.res_group[rs] == grp;
          const int G = D / L.VG;
          if (rb >= 0) {
            const long hb = (long)h * (D * bits / 8);
#pragma unroll
            for (int q4 = 0; q4 < CPT / 4; ++q4) {
              const int ch = dcb * CPT + 4 * q4;
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
#pragma unroll
      for (int e = 0; e < CPT; ++e) {
        const _Float16 khi = (_Float16)kx[e];
        kt[dt * KS + dcb * CPT + e] = khi;
        ktl[dt * KS + dcb * CPT + e] = (_Float16)(kx[e] - (float)khi);
        vt[(dcb * CPT + e) * VS + dt] = (_Float16)vx[e];
      }
    }
    __syncthreads();

#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      f4_t s[2];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        s[kh] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NQK; ++j) {
          const h8_t kf = *(const h8_t*)&kt[(16 * kh + n) * KS + 32 * j + 8 * c];
          const h8_t kl = *(const h8_t*)&ktl[(16 * kh + n) * KS + 32 * j + 8 * c];
          s[kh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[rb][j], s[kh], 0, 0, 0);
          s[kh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qf[rb][j], s[kh], 0, 0, 0);
          if constexpr (QLO) s[kh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qfl[rb][j], s[kh], 0, 0, 0);
        }
      }
      float p[8];
      float mt = -__builtin_inff();
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kp = k0 + 16 * kh + 4 * c + i;
          const bool ok = kp < kv_end && kp < qlim[rb];
          const float v = ok ? s[kh][i] * a.scale_log2 : -__builtin_inff();
          p[4 * kh + i] = v;
          mt = fmaxf(mt, v);
        }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float m_new = fmaxf(m_run[rb], mt);
      const float m_safe = m_new == -__builtin_inff() ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[rb] - m_safe);
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = __builtin_amdgcn_exp2f(p[e] - m_safe);
        psum += p[e];
      }
      l_lane[rb] = l_lane[rb] * alpha + psum;
      m_run[rb] = m_new;
      h8_t pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = (_Float16)p[e];
#pragma unroll
      for (int j = 0; j < NPV; ++j) {
        const _Float16* vr = &vt[(16 * j + n) * VS];
        const h4_t lo = *(const h4_t*)&vr[4 * c];
        const h4_t hi = *(const h4_t*)&vr[16 + 4 * c];
        const h8_t vf = h8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc[rb][j] *= alpha;
        acc[rb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pb, acc[rb][j], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float l = l_lane[rb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (!rvalid[rb]) continue;
    const int r = 16 * RB * wave + 16 * rb + n;
    const long ob = (q_row0 + r / gqa) * a.o_s0 + (long)(h * gqa + r % gqa) * a.o_s1;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (a.lse && c == 0) a.lse[(q_row0 + r / gqa) * a.hq + h * gqa + r % gqa] = l > 0.f ? m_run[rb] + __log2f(l) : -__builtin_inff();
#pragma unroll
    for (int j = 0; j < NPV; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) st(a.out, a.out_dtype, ob + 16 * j + 4 * c + i, acc[rb][j][i] * inv);
    }
  }
}

hipError_t launch_prefill(const PrefillArgs& a, long n_tiles, hipStream_t s) {
  const dim3 grid((unsigned)n_tiles, (unsigned)a.L.H);
  const bool qlo = a.q_dtype == ECHOKV_F32;
  if (a.L.D == 128) {
    if (qlo) hipLaunchKernelGGL((prefill_kernel<128, true, 2>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((prefill_kernel<128, false, 2>), grid, dim3(256), 0, s, a);
  } else if (a.L.D == 64) {
    if (qlo) hipLaunchKernelGGL((prefill_kernel<64, true, 2>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((prefill_kernel<64, false, 2>), grid, dim3(256), 0, s, a);
  } else if (a.L.D == 256) {
    if (qlo) hipLaunchKernelGGL((prefill_kernel<256, true, 1>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((prefill_kernel<256, false, 1>), grid, dim3(256), 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ek
