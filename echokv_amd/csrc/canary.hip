// Canary probe (echokv_vllm/canary.py:59-89) on gfx950: per layer and tier b,
// delta_b = mean over query rows and heads of KL(softmax(q K~_b^T s) || softmax(q K_ref^T s)),
// K~_b = per-channel storage round trip of the K_ref keys over whole k_group
// groups (oldest-first; the oldest window mod k_group keys are dropped).
//
// One workgroup per layer. For each KV head the (<= 64) keys are staged in LDS
// in float32 together with their round trip at every tier; then one wave per
// variant (reference + tiers) computes one query row's logits, lane j = key j,
// and the log-softmax / KL reductions are wave reductions. Everything is
// float32; it runs once per canary interval over <= 8 query rows.
#include "args.h"

namespace ek {



__device__ __forceinline__ float wave_max(float v) {
  for (int m = 32; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__global__ __launch_bounds__(256) void canary_kernel(CanaryArgs a) {
  // Key rows padded by one float: lane j reads row j, and unpadded rows of
  // kCanaryMaxD floats would put every lane's read in the same LDS bank.
  __shared__ float kv[1 + kCanaryMaxTiers][kCanaryMaxKeys][kCanaryMaxD + 1];
  __shared__ float lref[2][kCanaryMaxKeys];  // double-buffered by query row: one barrier per row
  const int layer = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int w = (a.window / a.kg) * a.kg;
  const int first = a.window - w;
  const int rep = a.hq / a.h;
  float kl = 0.f;  // wave t+1 accumulates tier t
  for (int h = 0; h < a.h; ++h) {
    __syncthreads();
    for (int i = tid; i < w * a.d; i += 256) {
      const int j = i / a.d, dd = i % a.d;
      kv[0][j][dd] = a.kref[layer * a.k_sl + (long)(first + j) * a.k_s0 + (long)h * a.k_s1 + dd];
    }
    __syncthreads();
    // Round trip per tier: one thread per (tier, channel, group).
    const int ngrp = w / a.kg;
    for (int i = tid; i < a.nbits * a.d * ngrp; i += 256) {
      const int t = i / (a.d * ngrp), r = i % (a.d * ngrp);
      const int dd = r % a.d, gi = r / a.d;
      const int bits = (a.bits_packed >> (8 * t)) & 0xff;
      float mn = __builtin_inff(), mx = -__builtin_inff();
      for (int p = 0; p < a.kg; ++p) {
        const float x = kv[0][gi * a.kg + p][dd];
        mn = fminf(mn, x);
        mx = fmaxf(mx, x);
      }
      _Float16 s16, m16;
      float s, m;
      group_stats(mn, mx, bits, s16, m16, s, m);
      for (int p = 0; p < a.kg; ++p) {
        const float x = kv[0][gi * a.kg + p][dd];
        kv[1 + t][gi * a.kg + p][dd] = (float)quant_code(x, m, s, bits) * s + m;
      }
    }
    __syncthreads();  // the round trips are staged
    int buf = 0;
    for (int qh = h * rep; qh < (h + 1) * rep; ++qh) {
      for (int r = 0; r < a.nq; ++r, buf ^= 1) {
        // The query row is the same for every lane: read 16 channels at a time
        // with wave-uniform (scalar) loads, no LDS staging or barrier.
        const long qb = layer * a.q_sl + (long)r * a.q_s0 + (long)qh * a.q_s1;
        float logit = -__builtin_inff();
        if (wave <= a.nbits && lane < w) {
          float acc = 0.f;
          int d0 = 0;
          for (; d0 + 16 <= a.d; d0 += 16) {
            float qv[16];
            ld_n<16>(a.q, a.q_dtype, qb + d0, qv);
#pragma unroll
            for (int e = 0; e < 16; ++e) acc += qv[e] * kv[wave][lane][d0 + e];
          }
          for (; d0 < a.d; ++d0) acc += ld(a.q, a.q_dtype, qb + d0) * kv[wave][lane][d0];  // head size not a multiple of 16
          logit = acc * a.scale;
        }
        float lsm = 0.f;
        if (wave <= a.nbits) {
          const float mx = wave_max(logit);
          const float e = lane < w ? expf(logit - mx) : 0.f;
          const float lse = mx + logf(wave_sum(e));
          lsm = logit - lse;
          if (wave == 0 && lane < w) lref[buf][lane] = lsm;
        }
        __syncthreads();
        if (wave >= 1 && wave <= a.nbits) {
          const float term = lane < w ? expf(lsm) * (lsm - lref[buf][lane]) : 0.f;
          const float s = wave_sum(term);
          kl += s;
        }
      }
    }
  }
  if (wave >= 1 && wave <= a.nbits && lane == 0) {
    const float mean = kl / (float)(a.nq * a.hq);
    a.out[layer * a.nbits + (wave - 1)] = fmaxf(mean, 0.f);
  }
}

hipError_t launch_canary(const CanaryArgs& a, int num_layers, hipStream_t s) {
  hipLaunchKernelGGL(canary_kernel, dim3((unsigned)num_layers), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace ek
