// Canary probe (echokv_vllm/canary.py:59-89) on gfx950: per layer and tier b,
// delta_b = mean over query rows and heads of KL(softmax(q K~_b^T s) || softmax(q K_ref^T s)),
// K~_b = per-channel storage round trip of the K_ref keys over whole k_group
// groups (oldest-first; the oldest window mod k_group keys are dropped).
//
// One workgroup per (layer, KV head): it scores the rep = Hq / H query heads of
// that KV head for all nq query rows. The window's keys are staged in LDS a chunk
// (64 keys; 32 above head size 128) at a time, in float32 together with their
// round trip at every tier, so any window length fits. One wave per variant
// (reference + tiers) computes one row's logits, lane j = key j. Per row the
// softmax statistics run online over the chunks against the reference's running
// max m:  s_v = sum exp(x_v - m),  u_b = sum exp(x_b - m) (x_b - x_ref), so that
// KL_b = u_b / s_b - log(s_b / s_ref) (no difference of two large log-sum-exps).
// Each workgroup writes its KL sums per tier; a second kernel adds the heads of
// a layer in order (deterministic) and takes the mean. Everything is float32.
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

// LDS layout of one workgroup (dynamic): keys [V][C][D + 1] (rows padded by one
// float so lane j reading row j hits its own bank), the reference logits of the
// row being scored [2][C] (double-buffered by row), the row max [2][2] (old,
// new), and the per-row running state [V][rows][2] (s, u).
struct CanaryLds {
  int C, D, V, rows;
  __host__ __device__ size_t keys() const { return (size_t)V * C * (D + 1); }
  __host__ __device__ size_t bytes() const { return 4 * (keys() + 2 * C + 4 + (size_t)V * rows * 2 + rows); }
};

__host__ __device__ inline int canary_chunk(int d) { return d <= 128 ? 64 : 32; }

__global__ __launch_bounds__(256) void canary_kernel(CanaryArgs a) {
  extern __shared__ float lds[];
  const int layer = blockIdx.x / a.h, h = blockIdx.x % a.h;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int rep = a.hq / a.h;
  const int rows = rep * a.nq;
  const CanaryLds L{canary_chunk(a.d), a.d, 1 + a.nbits, rows};
  float* kv = lds;                                  // [V][C][D + 1]
  float* lref = kv + L.keys();                      // [2][C]
  float* mrow = lref + 2 * L.C;                     // [2][2]: old, new max of the row
  float* st = mrow + 4;                             // [V][rows][2]: s, u
  float* mrun = st + (size_t)L.V * rows * 2;        // [rows]: the reference's running max
  const int w = (a.window / a.kg) * a.kg;
  const int first = a.window - w;
  const long kbase = layer * a.k_sl + (long)h * a.k_s1;
  const int D1 = a.d + 1;
  for (int i = tid; i < L.V * rows * 2; i += 256) st[i] = 0.f;
  for (int i = tid; i < rows; i += 256) mrun[i] = -__builtin_inff();

  int buf = 0;
  for (int c0 = 0; c0 < w; c0 += L.C) {
    const int nk = w - c0 < L.C ? w - c0 : L.C;
    __syncthreads();  // the previous chunk's keys are no longer read
    for (int i = tid; i < nk * a.d; i += 256) {
      const int j = i / a.d, dd = i % a.d;
      kv[j * D1 + dd] = a.kref[kbase + (long)(first + c0 + j) * a.k_s0 + dd];
    }
    __syncthreads();
    // Round trip per tier: one thread per (tier, channel, group touching the chunk).
    // A group inside the chunk takes its stats from LDS, a longer one from memory.
    const int g0 = c0 / a.kg, g1 = (c0 + nk - 1) / a.kg;
    const int ng = g1 - g0 + 1;
    for (int i = tid; i < a.nbits * a.d * ng; i += 256) {
      const int t = i / (a.d * ng), r = i % (a.d * ng);
      const int dd = r % a.d, g = g0 + r / a.d;
      const int bits = (a.bits_packed >> (8 * t)) & 0xff;
      float mn = __builtin_inff(), mx = -__builtin_inff();
      const bool in_chunk = g * a.kg >= c0 && (g + 1) * a.kg <= c0 + nk;
      for (int p = 0; p < a.kg; ++p) {
        const int k = g * a.kg + p;  // key index within the scored window
        const float x = in_chunk ? kv[(k - c0) * D1 + dd] : a.kref[kbase + (long)(first + k) * a.k_s0 + dd];
        mn = fminf(mn, x);
        mx = fmaxf(mx, x);
      }
      _Float16 s16, m16;
      float s, m;
      group_stats(mn, mx, bits, s16, m16, s, m);
      const int lo = g * a.kg > c0 ? g * a.kg - c0 : 0;
      const int hi = (g + 1) * a.kg - c0 < nk ? (g + 1) * a.kg - c0 : nk;
      for (int j = lo; j < hi; ++j) {
        const float x = kv[j * D1 + dd];
        kv[(size_t)(1 + t) * L.C * D1 + j * D1 + dd] = (float)quant_code(x, m, s, bits) * s + m;
      }
    }
    __syncthreads();  // the chunk's round trips are staged

    for (int row = 0; row < rows; ++row, buf ^= 1) {
      const int qh = h * rep + row / a.nq, r = row % a.nq;
      const long qb = layer * a.q_sl + (long)r * a.q_s0 + (long)qh * a.q_s1;
      const bool active = wave < L.V;
      float x = -__builtin_inff();
      if (active && lane < nk) {
        // The query row is the same for every lane: wave-uniform loads.
        const float* krow = kv + (size_t)wave * L.C * D1 + lane * D1;
        float acc = 0.f;
        int d0 = 0;
        for (; d0 + 16 <= a.d; d0 += 16) {
          float qv[16];
          ld_n<16>(a.q, a.q_dtype, qb + d0, qv);
#pragma unroll
          for (int e = 0; e < 16; ++e) acc += qv[e] * krow[d0 + e];
        }
        for (; d0 < a.d; ++d0) acc += ld(a.q, a.q_dtype, qb + d0) * krow[d0];  // head size not a multiple of 16
        x = acc * a.scale;
      }
      if (wave == 0) {  // the reference: running max and sum; publish its logits
        const float m_old = mrun[row];
        const float m_new = fmaxf(m_old, wave_max(x));
        const float e = lane < nk ? expf(x - m_new) : 0.f;
        const float se = wave_sum(e);
        if (lane < nk) lref[buf * L.C + lane] = x;
        if (lane == 0) {
          mrow[2 * buf] = m_old;
          mrow[2 * buf + 1] = m_new;
          mrun[row] = m_new;
          float* sv = st + (size_t)row * 2;
          sv[0] = sv[0] * expf(m_old - m_new) + se;
        }
      }
      __syncthreads();
      if (wave >= 1 && active) {
        const float m_old = mrow[2 * buf], m_new = mrow[2 * buf + 1];
        const float e = lane < nk ? expf(x - m_new) : 0.f;
        const float du = lane < nk ? e * (x - lref[buf * L.C + lane]) : 0.f;
        const float se = wave_sum(e), su = wave_sum(du);
        if (lane == 0) {
          float* sv = st + ((size_t)wave * rows + row) * 2;
          const float f = expf(m_old - m_new);  // m_old = -inf on the first chunk: f = 0
          sv[0] = sv[0] * f + se;
          sv[1] = sv[1] * f + su;
        }
      }
    }
  }
  __syncthreads();
  if (wave >= 1 && wave < L.V) {
    float kl = 0.f;
    for (int row = lane; row < rows; row += 64) {
      const float* sv = st + ((size_t)wave * rows + row) * 2;
      const float s_ref = st[(size_t)row * 2];
      kl += sv[1] / sv[0] - logf(sv[0] / s_ref);
    }
    kl = wave_sum(kl);
    if (lane == 0) a.partial[((long)layer * a.h + h) * a.nbits + (wave - 1)] = kl;
  }
}

// out[layer][t] = max(sum over KV heads of the partial sums / (nq * Hq), 0), heads in order.
__global__ __launch_bounds__(64) void canary_reduce_kernel(CanaryArgs a, int num_layers) {
  const int i = blockIdx.x * 64 + threadIdx.x;
  if (i >= num_layers * a.nbits) return;
  const int layer = i / a.nbits, t = i % a.nbits;
  float s = 0.f;
  for (int h = 0; h < a.h; ++h) s += a.partial[((long)layer * a.h + h) * a.nbits + t];
  a.out[i] = fmaxf(s / (float)(a.nq * a.hq), 0.f);
}

size_t canary_lds_bytes(int d, int nbits, int rows) {
  return CanaryLds{canary_chunk(d), d, 1 + nbits, rows}.bytes();
}

hipError_t launch_canary(const CanaryArgs& a, int num_layers, hipStream_t s) {
  const size_t lds = canary_lds_bytes(a.d, a.nbits, (a.hq / a.h) * a.nq);
  static std::atomic<uint64_t> attr_done{0};
  hipError_t e = ensure_lds_limit((const void*)canary_kernel, (int)lds, &attr_done);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(canary_kernel, dim3((unsigned)(num_layers * a.h)), dim3(256), lds, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(canary_reduce_kernel, dim3((unsigned)((num_layers * a.nbits + 63) / 64)), dim3(64), 0, s, a,
                     num_layers);
  return hipGetLastError();
}

}  // namespace ek
