// Paged decode attention for the layouts the MFMA decode kernels do not take
// (echokv_vllm/kernels/decode.py:95-129, the reference's PyTorch path for shapes
// its Triton kernel refuses): head sizes other than 64 / 128 / 256 (any multiple
// of 4 up to 256), V groups under D / 16 channels (at head size 256: outside 8 to
// 128), K groups under 16, block sizes or K groups that are not powers of two,
// more than 4 chunks per page.
//
// One workgroup per (sequence, KV head, split) in fp32 arithmetic, the split
// schedule of the MFMA kernels (splits of max(blocks_per_split, ceil(blocks /
// num_splits)) blocks, so a sequence's result does not depend on its batch) and
// the same workspace rows: acc [S, Hq, splits, D] unnormalized, ml (running max
// in log2 units, sum). Per tile of 64 keys:
//   - 64 threads locate their token (block, chunk row, tier from the header,
//     residual row when the token's K group is the block's open one);
//   - 4 threads per token score it against the pass's query heads (a quarter of
//     the channels each, reduced by two lane swaps);
//   - one wave per 4 query heads runs the online softmax over the tile;
//   - each thread owns one channel of O for a share of the tile's tokens.
// Each token is dequantized as the reference's gather does: K codes with the
// group's per-channel (scale, min), or the residual row for the open group; V
// codes with the token's per-group (scale, min); a chunk id outside the layer's
// pages reads as zeros. Block ids outside the layer are left out.
#include "args.h"

namespace ek {
namespace {

constexpr int kAnyThreads = 256;
constexpr int kAnyTile = 64;  // keys per tile
constexpr int kAnyCols = 16;  // query heads per pass (DecodeArgs::gs <= 16)

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

__global__ __launch_bounds__(kAnyThreads) void decode_any_kernel(DecodeArgs a) {
  const Lay& L = a.L;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const long wg = blockIdx.x;
  const int sp = (int)(wg % a.num_splits);
  const long sh = wg / a.num_splits;
  const int h = (int)(sh % L.H);
  const long seq = sh / L.H;
  const long seq_len = a.lens[seq];
  if (seq_len <= 0) return;
  const long n_blocks = (seq_len + L.BS - 1) / L.BS;
  const long per = (n_blocks + a.num_splits - 1) / a.num_splits;
  const long bps = a.bps > per ? a.bps : per;
  const long b0 = sp * bps;
  if (b0 >= n_blocks) return;
  const long t_begin = b0 * L.BS;
  const long t_end = (b0 + bps) * L.BS < seq_len ? (b0 + bps) * L.BS : seq_len;

  __shared__ __align__(16) float qs[kAnyCols * kMaxAnyD];  // the pass's queries (scaled); at the end, O's parts
  __shared__ float ps[kAnyCols][kAnyTile];   // scores, then probabilities
  __shared__ float alpha[kAnyCols];
  __shared__ long rbs[kAnyTile];   // token row base; -1: chunk id outside the pages; -2: left out
  __shared__ long pbs[kAnyTile];   // page base of the token's block
  __shared__ long kres[kAnyTile];  // residual element of the token's K row; -1: K from codes
  __shared__ int offs[kAnyTile];
  __shared__ int bits_s[kAnyTile];

  const int D = L.D, gs = a.gs, quads = D / 4, G = D / L.VG;
  const long q_row = a.q_rows ? a.q_rows[seq] : seq;
  const long bt_row = a.bt_rows ? a.bt_rows[seq] : seq;
  const int qh0 = h * a.gqa + a.g0;
  for (int i = tid; i < gs * D; i += kAnyThreads) {
    const int g = i / D, d = i - g * D;
    qs[i] = ld(a.q, a.q_dtype, q_row * a.q_s0 + (long)(qh0 + g) * a.q_s1 + d) * a.scale_log2;
  }

  float m_run[4], l_run[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -__builtin_inff();
    l_run[i] = 0.f;
  }
  const int NT = kAnyThreads / D;  // token shares of the PV phase
  const int r = tid / D, d = tid - r * D;
  float o[kAnyCols];
#pragma unroll
  for (int g = 0; g < kAnyCols; ++g) o[g] = 0.f;

  for (long t0 = t_begin; t0 < t_end; t0 += kAnyTile) {
    __syncthreads();  // the previous tile's PV phase is done with ps and the token rows
    if (tid < kAnyTile) {
      const long pos = t0 + tid;
      long rb = -2, pb = 0, kr = -1;
      int off = 0, bits = 2;
      if (pos < t_end) {
        const long b = pos / L.BS;
        off = (int)(pos - b * L.BS);
        const long blk = a.bt[bt_row * a.bt_s0 + b];
        if (blk >= 0 && blk < L.nb) {
          pb = blk * L.stride;
          bits = tier_of(a.pages[pb]);
          rb = row_base(a.pages, L, blk, off, bits);
          const long rs = a.block_res[blk];
          if (rs >= 0 && rs < a.res.rows && a.res_group[rs] == off / L.KG)
            kr = rs * a.res.s0 + (long)(off % L.KG) * a.res.s1 + (long)h * a.res.s2;
        }
      }
      rbs[tid] = rb;
      pbs[tid] = pb;
      kres[tid] = kr;
      offs[tid] = off;
      bits_s[tid] = bits;
    }
    __syncthreads();

    // Scores: token j, channel quads p, p + 4, ...
    {
      const int j = tid >> 2, p = tid & 3;
      float s[kAnyCols];
#pragma unroll
      for (int g = 0; g < kAnyCols; ++g) s[g] = 0.f;
      const long rb = rbs[j];
      if (rb >= 0) {
        const long kr = kres[j];
        const int bits = bits_s[j];
        const uint8_t* kp = a.pages + rb + (long)h * (D * bits / 8);
        const long se = pbs[j] + 2 * (((long)(offs[j] / L.KG) * L.H + h) * D);
        for (int c = p; c < quads; c += 4) {
          float k[4];
          if (kr >= 0) {
            ld4(a.res.ptr, a.res.dtype, kr + 4 * c, k);
          } else {
            const uint32_t kc = load_codes4(kp + c * (bits / 2), bits);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float ks = (float)*f16p(a.pages, se + L.o_ks + 2 * (4 * c + e));
              const float km = (float)*f16p(a.pages, se + L.o_km + 2 * (4 * c + e));
              k[e] = code_at(kc, e, bits) * ks + km;
            }
          }
#pragma unroll
          for (int g = 0; g < kAnyCols; ++g) {
            if (g < gs) {
              const float4 q = *(const float4*)&qs[g * D + 4 * c];
              s[g] += q.x * k[0] + q.y * k[1] + q.z * k[2] + q.w * k[3];
            }
          }
        }
      }
#pragma unroll
      for (int g = 0; g < kAnyCols; ++g) {
        s[g] += __shfl_xor(s[g], 1, 64);
        s[g] += __shfl_xor(s[g], 2, 64);
      }
      if (p == 0) {
#pragma unroll
        for (int g = 0; g < kAnyCols; ++g)
          if (g < gs) ps[g][j] = rb == -2 ? -__builtin_inff() : s[g];
      }
    }
    __syncthreads();

    // Online softmax: wave wv owns query heads wv, wv + 4, wv + 8, wv + 12.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = wv + 4 * i;
      if (g < gs) {
        const float x = ps[g][lane];
        const float m_new = fmaxf(m_run[i], wave_max(x));
        const bool none = m_new == -__builtin_inff();
        const float pr = none ? 0.f : __builtin_amdgcn_exp2f(x - m_new);
        const float al = none ? 1.f : __builtin_amdgcn_exp2f(m_run[i] - m_new);
        l_run[i] = l_run[i] * al + wave_sum(pr);
        m_run[i] = m_new;
        ps[g][lane] = pr;
        if (lane == 0) alpha[g] = al;
      }
    }
    __syncthreads();

    // O: channel d, tokens r, r + NT, ...
    if (r < NT) {
#pragma unroll
      for (int g = 0; g < kAnyCols; ++g)
        if (g < gs) o[g] *= alpha[g];
      for (int j = r; j < kAnyTile; j += NT) {
        const long rb = rbs[j];
        if (rb < 0) continue;  // left out, or a chunk id outside the pages (V reads as 0)
        const int bits = bits_s[j];
        const long vb = rb + (long)(L.H + h) * (D * bits / 8) + ((d * bits) >> 3);
        const float code = (float)((a.pages[vb] >> ((d * bits) & 7)) & ((1u << bits) - 1u));
        const long ve = ((long)offs[j] * L.H + h) * G + d / L.VG;
        const float vs = (float)*f16p(a.pages, pbs[j] + L.o_vs + 2 * ve);
        const float vm = (float)*f16p(a.pages, pbs[j] + L.o_vm + 2 * ve);
        const float v = code * vs + vm;
#pragma unroll
        for (int g = 0; g < kAnyCols; ++g)
          if (g < gs) o[g] += ps[g][j] * v;
      }
    }
  }

  // Sum O's token shares (qs is free now), then write the split's rows.
  __syncthreads();
  if (r < NT) {
#pragma unroll
    for (int g = 0; g < kAnyCols; ++g)
      if (g < gs) qs[(r * gs + g) * D + d] = o[g];
  }
  __syncthreads();
  const long row0 = (seq * a.hq + qh0) * a.num_splits + sp;  // + g * num_splits for query head g
  for (int i = tid; i < gs * D; i += kAnyThreads) {
    const int g = i / D, dd = i - g * D;
    float x = 0.f;
    for (int rr = 0; rr < NT; ++rr) x += qs[(rr * gs + g) * D + dd];
    a.acc[(row0 + (long)g * a.num_splits) * D + dd] = x;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int g = wv + 4 * i;
    if (g < gs && lane == 0) {
      const long row = row0 + (long)g * a.num_splits;
      a.ml[row * 2] = m_run[i];
      a.ml[row * 2 + 1] = l_run[i];
    }
  }
}

// Log-sum-exp merge of a row's splits (any D <= 256): one wave per (sequence, query head).
__global__ __launch_bounds__(256) void merge_any_kernel(MergeArgs a) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);  // seq * hq + head
  if (row >= a.rows) return;
  const long seq = row / a.hq;
  const int head = (int)(row % a.hq);
  if (head % a.gqa < a.g0 || head % a.gqa >= a.g0 + a.gs) return;  // another pass's query heads
  const long seq_len = a.lens[seq];
  if (seq_len <= 0) return;
  const long n_blocks = (seq_len + a.BS - 1) / a.BS;
  const long per = (n_blocks + a.num_splits - 1) / a.num_splits;
  const long bps = a.bps > per ? a.bps : per;
  const int used = (int)((n_blocks + bps - 1) / bps);
  const long base = row * a.num_splits;
  const int D = a.D;
  float m = -__builtin_inff();
  for (int s = lane; s < used; s += 64) m = fmaxf(m, a.ml[(base + s) * 2]);
  m = wave_max(m);
  float den = 0.f, num[kMaxAnyD / 64];
#pragma unroll
  for (int e = 0; e < kMaxAnyD / 64; ++e) num[e] = 0.f;
  for (int s = 0; s < used; ++s) {
    const float w = __builtin_amdgcn_exp2f(a.ml[(base + s) * 2] - m);
    den += a.ml[(base + s) * 2 + 1] * w;
    const float* src = a.acc + (base + s) * D;
#pragma unroll
    for (int e = 0; e < kMaxAnyD / 64; ++e)
      if (lane + 64 * e < D) num[e] += src[lane + 64 * e] * w;
  }
  const long o_row = a.q_rows ? a.q_rows[seq] : seq;
#pragma unroll
  for (int e = 0; e < kMaxAnyD / 64; ++e)
    if (lane + 64 * e < D) st(a.out, a.out_dtype, o_row * a.o_s0 + head * a.o_s1 + lane + 64 * e, num[e] / den);
}

// Chunked prefill for the same layouts (echokv_vllm/kernels/prefill.py:210-236, the
// reference's gather + bottom-right causal SDPA): one workgroup per (tile of
// query tokens, KV head). Its columns are (token i, query head g) pairs, at most
// 16; column (i, g) sees keys < q_pos0 + i + 1 of its request's context. The
// keys stream once per tile in 64-key tiles exactly as in decode_any_kernel, and
// each column's row is normalized and written at the end.
__global__ __launch_bounds__(kAnyThreads) void prefill_any_kernel(PrefillArgs a) {
  const Lay& L = a.L;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int h = (int)(blockIdx.x % L.H);
  const int32_t* td = a.tiles + (long)(blockIdx.x / L.H) * 5;
  const long q_row0 = td[0];
  const int q_pos0 = td[2], ctx = td[3];
  const long bt_row = td[4];
  const int gs = a.gs;
  // The host sizes tiles to at most 16 columns; a larger tile is cut to its first
  // 16 / gs tokens rather than overrun the LDS rows.
  const int max_tok = kAnyCols / gs > 0 ? kAnyCols / gs : 1;
  const int n_tok = td[1] < max_tok ? td[1] : max_tok;
  const int n_cols = n_tok * gs;
  const long kv_end = q_pos0 + n_tok < ctx ? q_pos0 + n_tok : ctx;

  __shared__ __align__(16) float qs[kAnyCols * kMaxAnyD];
  __shared__ float ps[kAnyCols][kAnyTile];
  __shared__ float alpha[kAnyCols];
  __shared__ long rbs[kAnyTile], pbs[kAnyTile], kres[kAnyTile];
  __shared__ int offs[kAnyTile], bits_s[kAnyTile];

  const int D = L.D, quads = D / 4, G = D / L.VG;
  const int qh0 = h * a.gqa + a.g0;
  for (int i = tid; i < n_cols * D; i += kAnyThreads) {
    const int c = i / D, d = i - c * D;
    const int tok = c / gs, g = c - tok * gs;
    qs[i] = ld(a.q, a.q_dtype, (q_row0 + tok) * a.q_s0 + (long)(qh0 + g) * a.q_s1 + d) * a.scale_log2;
  }

  float m_run[4], l_run[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -__builtin_inff();
    l_run[i] = 0.f;
  }
  const int NT = kAnyThreads / D;
  const int r = tid / D, d = tid - r * D;
  float o[kAnyCols];
#pragma unroll
  for (int c = 0; c < kAnyCols; ++c) o[c] = 0.f;

  for (long t0 = 0; t0 < kv_end; t0 += kAnyTile) {
    __syncthreads();
    if (tid < kAnyTile) {
      const long pos = t0 + tid;
      long rb = -2, pb = 0, kr = -1;
      int off = 0, bits = 2;
      if (pos < kv_end) {
        const long b = pos / L.BS;
        off = (int)(pos - b * L.BS);
        const long blk = a.bt[bt_row * a.bt_s0 + b];
        if (blk >= 0 && blk < L.nb) {
          pb = blk * L.stride;
          bits = tier_of(a.pages[pb]);
          rb = row_base(a.pages, L, blk, off, bits);
          const long rs = a.block_res[blk];
          if (rs >= 0 && rs < a.res.rows && a.res_group[rs] == off / L.KG)
            kr = rs * a.res.s0 + (long)(off % L.KG) * a.res.s1 + (long)h * a.res.s2;
        }
      }
      rbs[tid] = rb;
      pbs[tid] = pb;
      kres[tid] = kr;
      offs[tid] = off;
      bits_s[tid] = bits;
    }
    __syncthreads();

    {
      const int j = tid >> 2, p = tid & 3;
      float s[kAnyCols];
#pragma unroll
      for (int c = 0; c < kAnyCols; ++c) s[c] = 0.f;
      const long rb = rbs[j];
      if (rb >= 0) {
        const long kr = kres[j];
        const int bits = bits_s[j];
        const uint8_t* kp = a.pages + rb + (long)h * (D * bits / 8);
        const long se = pbs[j] + 2 * (((long)(offs[j] / L.KG) * L.H + h) * D);
        for (int q4 = p; q4 < quads; q4 += 4) {
          float k[4];
          if (kr >= 0) {
            ld4(a.res.ptr, a.res.dtype, kr + 4 * q4, k);
          } else {
            const uint32_t kc = load_codes4(kp + q4 * (bits / 2), bits);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float ks = (float)*f16p(a.pages, se + L.o_ks + 2 * (4 * q4 + e));
              const float km = (float)*f16p(a.pages, se + L.o_km + 2 * (4 * q4 + e));
              k[e] = code_at(kc, e, bits) * ks + km;
            }
          }
#pragma unroll
          for (int c = 0; c < kAnyCols; ++c) {
            if (c < n_cols) {
              const float4 q = *(const float4*)&qs[c * D + 4 * q4];
              s[c] += q.x * k[0] + q.y * k[1] + q.z * k[2] + q.w * k[3];
            }
          }
        }
      }
#pragma unroll
      for (int c = 0; c < kAnyCols; ++c) {
        s[c] += __shfl_xor(s[c], 1, 64);
        s[c] += __shfl_xor(s[c], 2, 64);
      }
      if (p == 0) {
        const long pos = t0 + j;
#pragma unroll
        for (int c = 0; c < kAnyCols; ++c) {
          if (c < n_cols) {
            const long lim = q_pos0 + c / gs + 1;  // bottom-right causal: keys <= the query's position
            ps[c][j] = (rb == -2 || pos >= lim) ? -__builtin_inff() : s[c];
          }
        }
      }
    }
    __syncthreads();

#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = wv + 4 * i;
      if (c < n_cols) {
        const float x = ps[c][lane];
        const float m_new = fmaxf(m_run[i], wave_max(x));
        const bool none = m_new == -__builtin_inff();
        const float pr = none ? 0.f : __builtin_amdgcn_exp2f(x - m_new);
        const float al = none ? 1.f : __builtin_amdgcn_exp2f(m_run[i] - m_new);
        l_run[i] = l_run[i] * al + wave_sum(pr);
        m_run[i] = m_new;
        ps[c][lane] = pr;
        if (lane == 0) alpha[c] = al;
      }
    }
    __syncthreads();

    if (r < NT) {
#pragma unroll
      for (int c = 0; c < kAnyCols; ++c)
        if (c < n_cols) o[c] *= alpha[c];
      for (int j = r; j < kAnyTile; j += NT) {
        const long rb = rbs[j];
        if (rb < 0) continue;
        const int bits = bits_s[j];
        const long vb = rb + (long)(L.H + h) * (D * bits / 8) + ((d * bits) >> 3);
        const float code = (float)((a.pages[vb] >> ((d * bits) & 7)) & ((1u << bits) - 1u));
        const long ve = ((long)offs[j] * L.H + h) * G + d / L.VG;
        const float v = code * (float)*f16p(a.pages, pbs[j] + L.o_vs + 2 * ve) +
                        (float)*f16p(a.pages, pbs[j] + L.o_vm + 2 * ve);
#pragma unroll
        for (int c = 0; c < kAnyCols; ++c)
          if (c < n_cols) o[c] += ps[c][j] * v;
      }
    }
  }

  // Sum O's token shares, normalize, write each column's row.
  __syncthreads();
  if (r < NT) {
#pragma unroll
    for (int c = 0; c < kAnyCols; ++c)
      if (c < n_cols) qs[(r * n_cols + c) * D + d] = o[c];
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = wv + 4 * i;
      if (c < n_cols) alpha[c] = l_run[i] > 0.f ? 1.f / l_run[i] : 0.f;
    }
  }
  __syncthreads();
  for (int i = tid; i < n_cols * D; i += kAnyThreads) {
    const int c = i / D, dd = i - c * D;
    float x = 0.f;
    for (int rr = 0; rr < NT; ++rr) x += qs[(rr * n_cols + c) * D + dd];
    const int tok = c / gs, g = c - tok * gs;
    st(a.out, a.out_dtype, (q_row0 + tok) * a.o_s0 + (long)(qh0 + g) * a.o_s1 + dd, x * alpha[c]);
  }
}

}  // namespace

hipError_t launch_decode_any(const DecodeArgs& a, hipStream_t s) {
  const long wgs = a.num_seqs * a.L.H * a.num_splits;
  hipLaunchKernelGGL(decode_any_kernel, dim3((unsigned)wgs), dim3(kAnyThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_prefill_any(const PrefillArgs& a, long n_tiles, hipStream_t s) {
  hipLaunchKernelGGL(prefill_any_kernel, dim3((unsigned)(n_tiles * a.L.H)), dim3(kAnyThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_merge_any(const MergeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(merge_any_kernel, dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace ek
