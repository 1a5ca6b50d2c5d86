// Write-side and dequantization kernels of the tiered page store (gfx950).
//
// One workgroup of 256 threads per token row / K group / block; a thread owns
// four consecutive channels of one KV head, so a V group of VG channels is a
// segment of VG/4 lanes reduced with cross-lane shuffles (any other V group is
// scanned per group, store_v4), and every thread stores its four packed codes
// (1, 2 or 4 bytes) next to its neighbours' (coalesced). Numerics follow
// echokv_vllm/quant.py bit for bit: float32 extremes, fp16-rounded stats, IEEE
// division, round half to even.
#include "args.h"

namespace ek {

// V groups of 4 * 2^j channels are lane segments (seg_minmax); any other divisor
// of D (24, 12, 6, 3, 2, 1 channels at D 96, ...) is not. The same for every
// thread of a launch.
__device__ __forceinline__ bool v_segments(const Lay& L) {
  const int w = L.VG / 4;
  return L.VG % 4 == 0 && (w & (w - 1)) == 0;
}

// One token's V (head h, channels 4c..4c+3, values x) at `bits`: the group stats
// (written by the thread holding a group's first channel) and the packed codes at
// byte `vrow` (the token row's V side). With lane segments, (mn, mx) are the
// thread's group extremes already (seg_minmax over the wave); otherwise each
// channel's group is scanned from the source row, val(ch) = the row's channel ch,
// so a thread's channels may sit in up to four groups.
// quant.py:26-45 (quantize over groups of VG along the head dimension).
template <typename Val>
__device__ __forceinline__ void store_v4(const Lay& L, uint8_t* pages, long blk, long vrow, int off, int h, int c,
                                         const float x[4], int bits, float mn, float mx, Val val) {
  const int G = L.D / L.VG;
  const long sb = blk * L.stride;
  uint32_t q[4];
  if (v_segments(L)) {
    _Float16 s16, m16;
    float s, m;
    group_stats(mn, mx, bits, s16, m16, s, m);
    if ((4 * c) % L.VG == 0) {
      const long e = ((long)off * L.H + h) * G + (4 * c) / L.VG;
      *f16p(pages, sb + L.o_vs + 2 * e) = s16;
      *f16p(pages, sb + L.o_vm + 2 * e) = m16;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = quant_code(x[e], m, s, bits);
  } else {
    int gp = -1;
    float s = 1.f, m = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ch = 4 * c + e, g = ch / L.VG;
      if (g != gp) {  // a group starts here or at e == 0
        float gmn = val(g * L.VG), gmx = gmn;
        for (int j = g * L.VG + 1; j < (g + 1) * L.VG; ++j) {
          const float y = val(j);
          gmn = fminf(gmn, y);
          gmx = fmaxf(gmx, y);
        }
        _Float16 s16, m16;
        group_stats(gmn, gmx, bits, s16, m16, s, m);
        if (ch % L.VG == 0) {
          const long ve = ((long)off * L.H + h) * G + g;
          *f16p(pages, sb + L.o_vs + 2 * ve) = s16;
          *f16p(pages, sb + L.o_vm + 2 * ve) = m16;
        }
        gp = g;
      }
      q[e] = quant_code(x[e], m, s, bits);
    }
  }
  store_codes4(pages + vrow + (long)h * (L.D * bits / 8) + c * (bits / 2), pack4(q, bits), bits);
}


// ---------------------------------------------------------------------------
// write_tokens (echokv_vllm/kernels/write.py:29-36, 172-229)
// ---------------------------------------------------------------------------

// Token row t. res_here() says whether this workgroup stores the row's K to the
// residual (a fused step leaves that store to the workgroup finalizing the slot's
// old group); every thread calls it once, after the row's first loads are issued,
// so a caller may run a workgroup-wide vote in it.
template <typename ResHere>
__device__ __forceinline__ void write_token_row(const WriteTokArgs& a, long t, ResHere res_here) {
  const Lay& L = a.L;
  // The row's plan and its first pass's K / V words do not depend on one another:
  // they are requested together, before the slot is known (row t of key and value
  // exists whatever the slot), so the row costs two memory round trips.
  const long slot = a.tok[t];
  const long rslot = a.tok[a.tok_s0 + t];
  const int64_t sealed = a.tok[2 * a.tok_s0 + t];
  const long kidx = a.kref ? a.tok[3 * a.tok_s0 + t] : -1;
  const int quads = L.D / 4;
  const int items = L.H * quads;
  float x0[4] = {0.f, 0.f, 0.f, 0.f}, k0[4] = {0.f, 0.f, 0.f, 0.f};
  if ((int)threadIdx.x < items) {
    const int h = (int)threadIdx.x / quads, c = (int)threadIdx.x % quads;
    ld_n<4>(a.value, a.kv_dtype, t * a.v_s0 + h * a.v_s1 + 4 * c, x0);
    ld_n<4>(a.key, a.kv_dtype, t * a.k_s0 + h * a.k_s1 + 4 * c, k0);
  }
  if (slot < 0) return;
  const long blk = slot / L.BS;
  const int off = (int)(slot % L.BS);
  if (blk >= L.nb) return;
  const Hdr hd = load_hdr(a.pages, L, blk);
  bool rh = true;
  for (int base = 0; base < items; base += kThreads) {
    const int i = base + (int)threadIdx.x;
    const bool act = i < items;
    const int h = act ? i / quads : 0, c = act ? i % quads : 0;
    float x[4] = {x0[0], x0[1], x0[2], x0[3]}, k[4] = {k0[0], k0[1], k0[2], k0[3]};
    if (act && base > 0) {
      ld_n<4>(a.value, a.kv_dtype, t * a.v_s0 + h * a.v_s1 + 4 * c, x);
      ld_n<4>(a.key, a.kv_dtype, t * a.k_s0 + h * a.k_s1 + 4 * c, k);
    }
    _Float16 ks16[4], km16[4];  // the sealed group's stats (K codes under them)
    if (act && sealed != 0) {
      const long se = ((long)(off / L.KG) * L.H + h) * L.D + 4 * c;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ks16[e] = *f16p(a.pages, blk * L.stride + L.o_ks + 2 * (se + e));
        km16[e] = *f16p(a.pages, blk * L.stride + L.o_km + 2 * (se + e));
      }
    }
    if (base == 0) rh = res_here();  // uniform: every thread runs the first pass
    const int bits = tier_of(hd.tag);
    const long rb = row_base_h(L, blk, hd, off, bits);
    const int side = L.H * L.D * bits / 8;
    float mn = fminf(fminf(x[0], x[1]), fminf(x[2], x[3]));
    float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    // All lanes take part (uniform branch): segments never straddle `act`.
    if (v_segments(L)) seg_minmax(mn, mx, L.VG / 4);
    if (!act || rb < 0) continue;
    const long vsrc = t * a.v_s0 + h * a.v_s1;
    store_v4(L, a.pages, blk, rb + side, off, h, c, x, bits, mn, mx,
             [&](int ch) { return ld(a.value, a.kv_dtype, vsrc + ch); });

    // K: residual (open group), codes under the sealed stats, K_ref ring.
    if (rh && rslot >= 0 && rslot < a.res.rows)
      st_n<4>(a.res.ptr, a.res.dtype, rslot * a.res.s0 + (long)(off % L.KG) * a.res.s1 + h * a.res.s2 + 4 * c, k);
    if (sealed != 0) {
      uint32_t kq[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) kq[e] = quant_code(k[e], (float)km16[e], (float)ks16[e], bits);
      store_codes4(a.pages + rb + (long)h * (L.D * bits / 8) + c * (bits / 2), pack4(kq, bits), bits);
    }
    if (kidx >= 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) a.kref[kidx * a.kref_s0 + h * a.kref_s1 + 4 * c + e] = k[e];
    }
  }
}

__global__ __launch_bounds__(kThreads) void write_tokens_kernel(WriteTokArgs a) {
  write_token_row(a, blockIdx.x, [] { return true; });
}

// ---------------------------------------------------------------------------
// K-group quantization shared by finalize_k, seal and store_blocks: the group's
// n tokens of (head h, channels 4c..4c+3) come from `fetch(p, x)`; per-channel
// stats over the n tokens, then codes for each token at offset off0 + p.
// ---------------------------------------------------------------------------
template <typename Fetch>
__device__ __forceinline__ void quantize_k_group(const Lay& L, uint8_t* pages, long blk, int grp, int off0, int n, int bits, int h,
                                 int c, Fetch fetch) {
  // The group's tokens are held in registers 32 at a time: all their loads
  // (and the page header's) are in flight together, and a group of up to 32
  // tokens is read once -- the per-step groups (K group 16 or 32) cost two
  // or three dependent memory round trips instead of one per 8 tokens per pass.
  constexpr int kChunk = 32;
  const Hdr hd = load_hdr(pages, L, blk);
  float x[kChunk][4];
  float mn[4], mx[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mn[e] = __builtin_inff();
    mx[e] = -__builtin_inff();
  }
  for (int p0 = 0; p0 < n; p0 += kChunk) {
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      if (p0 + u < n) fetch(p0 + u, x[u]);
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      if (p0 + u < n) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          mn[e] = fminf(mn[e], x[u][e]);
          mx[e] = fmaxf(mx[e], x[u][e]);
        }
      }
    }
  }
  float s[4], m[4];
  const long se = ((long)grp * L.H + h) * L.D + 4 * c;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    _Float16 s16, m16;
    group_stats(mn[e], mx[e], bits, s16, m16, s[e], m[e]);
    *f16p(pages, blk * L.stride + L.o_ks + 2 * (se + e)) = s16;
    *f16p(pages, blk * L.stride + L.o_km + 2 * (se + e)) = m16;
  }
  for (int p0 = 0; p0 < n; p0 += kChunk) {
    if (n > kChunk) {  // a group over 32 tokens: the registers hold its last chunk
#pragma unroll
      for (int u = 0; u < kChunk; ++u)
        if (p0 + u < n) fetch(p0 + u, x[u]);
    }
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      if (p0 + u >= n) continue;
      const long rb = row_base_h(L, blk, hd, off0 + p0 + u, bits);
      if (rb < 0) continue;
      uint32_t q[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) q[e] = quant_code(x[u][e], m[e], s[e], bits);
      store_codes4(pages + rb + (long)h * (L.D * bits / 8) + c * (bits / 2), pack4(q, bits), bits);
    }
  }
}

// ---------------------------------------------------------------------------
// finalize_k (echokv_vllm/kernels/write.py:39-50, 232-287)
// ---------------------------------------------------------------------------

// The common case -- key and residual of one dtype, a group of at most 32
// tokens -- as straight-line code: every token's 4 values are loaded without
// a branch (the source is a select between this step's key row and the
// residual row; tokens past the group repeat its last one, which leaves the
// min / max unchanged), all loads in flight together; the block's chunk bases
// are computed once and rows are walked without divisions.
template <typename T>
__device__ __forceinline__ void finalize_group(const FinArgs a, const int64_t* row, long blk, int grp, long rs, int h,
                                               int c) {
  constexpr int kMax = 32;
  const Lay& L = a.L;
  const int n = L.KG;
  const Hdr hd = load_hdr(a.pages, L, blk);
  const T* key = (const T*)a.key;
  const T* res = (const T*)a.res.ptr;
  float x[kMax][4];
#pragma unroll
  for (int u = 0; u < kMax; ++u) {
    const int p = u < n ? u : n - 1;
    const long r = row[3 + p];
    const T* src = r >= 0 ? key + r * a.k_s0 + h * a.k_s1 + 4 * c
                          : res + rs * a.res.s0 + (long)p * a.res.s1 + h * a.res.s2 + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) x[u][e] = (float)src[e];
  }
  float mn[4], mx[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mn[e] = x[0][e];
    mx[e] = x[0][e];
#pragma unroll
    for (int u = 1; u < kMax; ++u) {
      mn[e] = fminf(mn[e], x[u][e]);
      mx[e] = fmaxf(mx[e], x[u][e]);
    }
  }
  const int bits = tier_of(hd.tag);
  float s[4], m[4];
  const long se = ((long)grp * L.H + h) * L.D + 4 * c;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    _Float16 s16, m16;
    group_stats(mn[e], mx[e], bits, s16, m16, s[e], m[e]);
    *f16p(a.pages, blk * L.stride + L.o_ks + 2 * (se + e)) = s16;
    *f16p(a.pages, blk * L.stride + L.o_km + 2 * (se + e)) = m16;
  }
  // Chunk j of the block: its own page's data for j = 0, pool chunk id[j - 1]
  // otherwise (-1: out of range, nothing stored there).
  long cb[4];
  cb[0] = blk * L.stride + L.o_data;
#pragma unroll
  for (int j = 1; j < 4; ++j) {
    const int id = hd.id(j - 1);
    const uint32_t page = (uint32_t)id / (uint32_t)L.KC, slot = (uint32_t)id % (uint32_t)L.KC;
    cb[j] = (id < 0 || (long)page >= L.nb) ? -1L : (long)page * L.stride + L.o_data + (long)slot * L.cb;
  }
  const int tpc = 2 * L.BS / bits;  // tokens per chunk
  const long rowb = 2L * L.H * L.D * bits / 8;
  const long within = (long)h * (L.D * bits / 8) + c * (bits / 2);
  int j = (grp * L.KG) / tpc, w = (grp * L.KG) % tpc;
#pragma unroll
  for (int u = 0; u < kMax; ++u) {
    if (u < n) {
      const long base = j == 0 ? cb[0] : (j == 1 ? cb[1] : (j == 2 ? cb[2] : cb[3]));
      if (base >= 0) {
        uint32_t q[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = quant_code(x[u][e], m[e], s[e], bits);
        store_codes4(a.pages + base + w * rowb + within, pack4(q, bits), bits);
      }
      if (++w == tpc) {
        w = 0;
        ++j;
      }
    }
  }
}

// Deferred residual stores of a fused step: token rows whose K goes to the slot
// a fin row releases, with the residual row each one writes.
struct Deferred {
  long t[kMaxDeferred];
  int row[kMaxDeferred];
  int n;
};

// Fin row f, one (head, quad) item per thread pass; after an item's reads (its
// stats and codes depend on them), the residual K stores of the token rows in
// `def` for the same item: a thread overwrites only residual words it has read.
__device__ __forceinline__ void finalize_row(const FinArgs& a, long f, const WriteTokArgs* w, const Deferred* def) {
  const Lay& L = a.L;
  const int64_t* row = a.fin + f * (3 + L.KG);
  const long blk = row[0];
  const int grp = (int)row[1];
  const long rs = row[2] < 0 ? 0 : row[2];
  const bool ok = blk >= 0 && blk < L.nb && grp >= 0 && grp < L.BS / L.KG && rs < a.res.rows;
  const int quads = L.D / 4;
  const bool same = a.kv_dtype == a.res.dtype && L.KG <= 32;
  const int n_def = def ? def->n : 0;
  for (int i = threadIdx.x; i < L.H * quads; i += kThreads) {
    const int h = i / quads, c = i % quads;
    if (!ok) {
    } else if (same && a.kv_dtype == ECHOKV_F16) {
      finalize_group<_Float16>(a, row, blk, grp, rs, h, c);
    } else if (same && a.kv_dtype == ECHOKV_F32) {
      finalize_group<float>(a, row, blk, grp, rs, h, c);
    } else {
      const int bits = tier_of(a.pages[blk * L.stride]);
      auto fetch = [&](int p, float x[4]) {
        const long r = row[3 + p];
        if (r >= 0) ld4(a.key, a.kv_dtype, r * a.k_s0 + h * a.k_s1 + 4 * c, x);
        else ld4(a.res.ptr, a.res.dtype, rs * a.res.s0 + (long)p * a.res.s1 + h * a.res.s2 + 4 * c, x);
      };
      quantize_k_group(L, a.pages, blk, grp, grp * L.KG, L.KG, bits, h, c, fetch);
    }
    for (int d = 0; d < n_def; ++d) {
      float k[4];
      ld_n<4>(w->key, w->kv_dtype, def->t[d] * w->k_s0 + h * w->k_s1 + 4 * c, k);
      st_n<4>(a.res.ptr, a.res.dtype, row[2] * a.res.s0 + (long)def->row[d] * a.res.s1 + h * a.res.s2 + 4 * c, k);
    }
  }
}

__global__ __launch_bounds__(kThreads) void finalize_k_kernel(FinArgs a) {
  const long f = blockIdx.x;
  if (f >= *a.fin_count) return;
  finalize_row(a, f, nullptr, nullptr);
}

// ---------------------------------------------------------------------------
// One step's writes in one launch (the pair finalize_k, write_tokens).
//
// Workgroups [0, fin_grid) take fin rows (rows at or past the device count do
// nothing), the rest token rows. The pair's order matters only where a token's K
// goes to a residual slot that a fin row of the step releases (the slot's old
// group completes now and is read from it): both sides see that from the plan
// itself -- fin row f's slot fin[f][2] equals the token's residual slot -- and
// that one store moves to the fin row's workgroup, after its reads; nothing waits
// on another workgroup.
//
// At decode shape a workgroup's time is a chain of dependent memory round trips
// (2-3 us each once the previous kernel has cycled the caches) plus instruction
// fetch, which starts cold every launch. So each workgroup issues every load that
// depends only on its row in a first round trip (fin rows f < fin_grid are all in
// the buffer; the count only says which are real), everything that depends on
// those in a second, and runs its per-token work as short loops: a fin row stages
// its group's values in LDS rather than in unrolled registers.
// ---------------------------------------------------------------------------

// Four consecutive channels of a 16-bit (uint2) or f32 (uint4) source, as stored.
template <int DT> struct Raw4 { using V = uint2; };
template <> struct Raw4<ECHOKV_F32> { using V = uint4; };

template <int DT>
__device__ __forceinline__ void raw4_to_f(const typename Raw4<DT>::V& r, float x[4]) {
  if constexpr (DT == ECHOKV_F32) {
    x[0] = __uint_as_float(r.x);
    x[1] = __uint_as_float(r.y);
    x[2] = __uint_as_float(r.z);
    x[3] = __uint_as_float(r.w);
  } else {
    const uint32_t wd[2] = {r.x, r.y};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t b = (uint16_t)(wd[e >> 1] >> (16 * (e & 1)));
      if constexpr (DT == ECHOKV_F16) x[e] = (float)__builtin_bit_cast(_Float16, b);
      else x[e] = bf16_to_f32(b);
    }
  }
}

constexpr int kStepScan = 8;  // token rows per thread whose loads one scan pass issues together

// Token rows of the step whose residual slot is rs (their K goes to the slot this
// fin row releases). The caller loaded row threadIdx.x's (slot, residual slot).
__device__ __forceinline__ void collect_deferred(const WriteTokArgs& a, long n_rows, long rs, long tslot, long tres,
                                                 Deferred& def) {
  auto add = [&](long t, long slot) {
    const int i = atomicAdd(&def.n, 1);  // LDS counter: at most k_group - 1 rows take a slot in a step
    if (i < kMaxDeferred) {
      def.t[i] = t;
      def.row[i] = (int)((slot % a.L.BS) % a.L.KG);
    }
  };
  if (tslot >= 0 && tres == rs) add(threadIdx.x, tslot);
  for (long t0 = kThreads + threadIdx.x; t0 < n_rows; t0 += (long)kThreads * kStepScan) {
    long sl[kStepScan], re[kStepScan];
#pragma unroll
    for (int k = 0; k < kStepScan; ++k) {
      const long t = t0 + (long)k * kThreads;
      sl[k] = t < n_rows ? a.tok[t] : -1;
      re[k] = t < n_rows ? a.tok[a.tok_s0 + t] : -1;
    }
#pragma unroll
    for (int k = 0; k < kStepScan; ++k)
      if (sl[k] >= 0 && re[k] == rs) add(t0 + (long)k * kThreads, sl[k]);
  }
}

// Round trip 1 of a fin row: its (block, group, residual slot), the device count
// and the step's token slots, then the deferred rows. Returns false when the row
// is past the count.
struct FinHead {
  long blk, rs;
  int grp;
};
__device__ __forceinline__ bool fin_prologue(const StepArgs& s, long f, Deferred& def, int64_t* grow,
                                             FinHead* head = nullptr) {
  const WriteTokArgs& a = s.w;
  const int64_t* row = s.fin + f * (3 + a.L.KG);
  const long count = *s.fin_count;
  const long rs = row[2];
  if (head) *head = FinHead{row[0], rs, (int)row[1]};
  if (grow && (int)threadIdx.x < a.L.KG) grow[threadIdx.x] = row[3 + threadIdx.x];
  const bool mine = (long)threadIdx.x < s.n_rows;
  const long tslot = mine ? a.tok[threadIdx.x] : -1;
  const long tres = mine ? a.tok[a.tok_s0 + threadIdx.x] : -1;
  if (threadIdx.x == 0) def.n = 0;
  __syncthreads();
  if (f >= count) return false;
  if (rs >= 0 && rs < a.res.rows) collect_deferred(a, s.n_rows, rs, tslot, tres, def);
  __syncthreads();
  if (def.n > kMaxDeferred) def.n = kMaxDeferred;  // not reached: the host checks k_group <= kMaxDeferred
  return true;
}

// Fin row f with key and residual of dtype DT: the group's values go through LDS
// (xs: [k_group][kThreads], each thread reads back only what it wrote).
template <int DT>
__device__ __forceinline__ void fin_staged(const StepArgs& s, long f, typename Raw4<DT>::V* xs, const Deferred& def,
                                           const int64_t* grow) {
  using V = typename Raw4<DT>::V;
  constexpr long esz = DT == ECHOKV_F32 ? 4 : 2;
  const WriteTokArgs& a = s.w;
  const Lay& L = a.L;
  const int KG = L.KG;
  const int64_t* row = s.fin + f * (3 + KG);
  const long blk = row[0];
  const int grp = (int)row[1];
  const long rs_raw = row[2];
  const long rs = rs_raw < 0 ? 0 : rs_raw;  // -1: every token of the group is in this step's key
  const bool ok = blk >= 0 && blk < L.nb && grp >= 0 && grp < L.BS / KG && rs < a.res.rows;
  const int n_def = def.n;
  const int quads = L.D / 4;
  const Hdr hd = load_hdr(a.pages, L, ok ? blk : 0);  // block 0 stands in for a bad row (nothing is stored)
  const char* key = (const char*)a.key;
  const char* res = (const char*)a.res.ptr;
  for (int i = threadIdx.x; i < L.H * quads; i += kThreads) {
    const int h = i / quads, c = i % quads;
    // Round trip 2: the group's values, and the first deferred rows' keys.
    float kd[2][4];
#pragma unroll
    for (int d = 0; d < 2; ++d)
      if (d < n_def) ld_n<4>(a.key, a.kv_dtype, def.t[d] * a.k_s0 + h * a.k_s1 + 4 * c, kd[d]);
    if (ok) {
      float mn[4], mx[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        mn[e] = __builtin_inff();
        mx[e] = -__builtin_inff();
      }
      for (int p0 = 0; p0 < KG; p0 += 16) {
        V v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int p = p0 + u;
          if (p < KG) {
            const long r = grow[p];
            const char* src = r >= 0 ? key + esz * (r * a.k_s0 + h * a.k_s1 + 4 * c)
                                     : res + esz * (rs * a.res.s0 + (long)p * a.res.s1 + h * a.res.s2 + 4 * c);
            v[u] = *(const V*)src;
          }
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int p = p0 + u;
          if (p < KG) {
            xs[p * kThreads + threadIdx.x] = v[u];
            float x[4];
            raw4_to_f<DT>(v[u], x);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              mn[e] = fminf(mn[e], x[e]);
              mx[e] = fmaxf(mx[e], x[e]);
            }
          }
        }
      }
      const int bits = tier_of(hd.tag);
      float sc[4], mi[4];
      const long se = ((long)grp * L.H + h) * L.D + 4 * c;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        _Float16 s16, m16;
        group_stats(mn[e], mx[e], bits, s16, m16, sc[e], mi[e]);
        *f16p(a.pages, blk * L.stride + L.o_ks + 2 * (se + e)) = s16;
        *f16p(a.pages, blk * L.stride + L.o_km + 2 * (se + e)) = m16;
      }
      // Chunk j of the block: its own page's data for j = 0, pool chunk id[j - 1]
      // otherwise (-1: out of range, nothing stored there).
      long cb[4];
      cb[0] = blk * L.stride + L.o_data;
#pragma unroll
      for (int j = 1; j < 4; ++j) {
        const int id = hd.id(j - 1);
        const uint32_t page = (uint32_t)id / (uint32_t)L.KC, slot = (uint32_t)id % (uint32_t)L.KC;
        cb[j] = (id < 0 || (long)page >= L.nb) ? -1L : (long)page * L.stride + L.o_data + (long)slot * L.cb;
      }
      const int tpc = 2 * L.BS / bits;  // tokens per chunk
      const long rowb = 2L * L.H * L.D * bits / 8;
      const long within = (long)h * (L.D * bits / 8) + c * (bits / 2);
      int j = (grp * KG) / tpc, w = (grp * KG) % tpc;
#pragma unroll 4
      for (int p = 0; p < KG; ++p) {
        const long base = j == 0 ? cb[0] : (j == 1 ? cb[1] : (j == 2 ? cb[2] : cb[3]));
        if (base >= 0) {
          float x[4];
          raw4_to_f<DT>(xs[p * kThreads + threadIdx.x], x);
          uint32_t q[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) q[e] = quant_code(x[e], mi[e], sc[e], bits);
          store_codes4(a.pages + base + w * rowb + within, pack4(q, bits), bits);
        }
        if (++w == tpc) {
          w = 0;
          ++j;
        }
      }
    }
    // Residual K of the deferred rows: this thread has read these words above.
    for (int d = 0; d < n_def; ++d) {
      float k[4];
      if (d < 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) k[e] = d == 0 ? kd[0][e] : kd[1][e];
      } else {
        ld_n<4>(a.key, a.kv_dtype, def.t[d] * a.k_s0 + h * a.k_s1 + 4 * c, k);
      }
      st_n<4>(a.res.ptr, a.res.dtype, rs_raw * a.res.s0 + (long)def.row[d] * a.res.s1 + h * a.res.s2 + 4 * c, k);
    }
  }
}

// Fin row f split over workgroups (StepArgs::fin_parts > 0): part `part` takes
// items [64 part, 64 part + 64) ((head, quad) pairs), and each item's K group is
// spread over the 4 lanes 16 apart (quarter r = lane / 16 holds positions
// r TPT .. r TPT + TPT - 1 in registers). The per-channel min / max meet by two
// lane swaps (min and max are exact, so the order does not matter), and each
// thread quantizes and stores its own positions: a group's codes cost TPT
// dependent divisions per thread, not k_group. The residual words of a deferred
// row are rewritten by the thread that read that position (if it read the
// residual there), after its read.
template <int DT, int TPT>
__device__ __forceinline__ void fin_split(const StepArgs& s, const FinHead& fh, int part, const Deferred& def,
                                          const int64_t* grow) {
  using V = typename Raw4<DT>::V;
  constexpr long esz = DT == ECHOKV_F32 ? 4 : 2;
  const WriteTokArgs& a = s.w;
  const Lay& L = a.L;
  const int KG = L.KG;  // = 4 * TPT
  const long blk = fh.blk;
  const int grp = fh.grp;
  const long rs_raw = fh.rs;
  const long rs = rs_raw < 0 ? 0 : rs_raw;  // -1: every token of the group is in this step's key
  const bool ok = blk >= 0 && blk < L.nb && grp >= 0 && grp < L.BS / KG && rs < a.res.rows;
  const int lane = threadIdx.x & 63, r = lane >> 4;
  const int quads = L.D / 4;
  const int i = part * 64 + (int)(threadIdx.x >> 6) * 16 + (lane & 15);
  const bool act = i < L.H * quads;  // whole 16-lane groups: every quarter of an item agrees
  const int h = act ? i / quads : 0, c = act ? i % quads : 0;
  const Hdr hd = load_hdr(a.pages, L, ok ? blk : 0);  // block 0 stands in for a bad row (nothing is stored)
  const char* key = (const char*)a.key;
  const char* res = (const char*)a.res.ptr;
  float x[TPT][4];
  float mn[4], mx[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mn[e] = __builtin_inff();
    mx[e] = -__builtin_inff();
  }
  if (act && ok) {
    V v[TPT];
#pragma unroll
    for (int u = 0; u < TPT; ++u) {
      const int p = r * TPT + u;
      const long t = grow[p];
      const char* src = t >= 0 ? key + esz * (t * a.k_s0 + h * a.k_s1 + 4 * c)
                               : res + esz * (rs * a.res.s0 + (long)p * a.res.s1 + h * a.res.s2 + 4 * c);
      v[u] = *(const V*)src;
    }
#pragma unroll
    for (int u = 0; u < TPT; ++u) {
      raw4_to_f<DT>(v[u], x[u]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        mn[e] = fminf(mn[e], x[u][e]);
        mx[e] = fmaxf(mx[e], x[u][e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {  // the item's four quarters: lanes l, l ^ 16, l ^ 32, l ^ 48
    mn[e] = fminf(mn[e], __shfl_xor(mn[e], 16, 64));
    mx[e] = fmaxf(mx[e], __shfl_xor(mx[e], 16, 64));
    mn[e] = fminf(mn[e], __shfl_xor(mn[e], 32, 64));
    mx[e] = fmaxf(mx[e], __shfl_xor(mx[e], 32, 64));
  }
  if (act && ok) {
    const int bits = tier_of(hd.tag);
    float sc[4], mi[4];
    const long se = ((long)grp * L.H + h) * L.D + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      _Float16 s16, m16;
      group_stats(mn[e], mx[e], bits, s16, m16, sc[e], mi[e]);
      if (r == 0) {
        *f16p(a.pages, blk * L.stride + L.o_ks + 2 * (se + e)) = s16;
        *f16p(a.pages, blk * L.stride + L.o_km + 2 * (se + e)) = m16;
      }
    }
    long cb[4];  // chunk j of the block (its own page's data for j = 0; -1: out of range)
    cb[0] = blk * L.stride + L.o_data;
#pragma unroll
    for (int j = 1; j < 4; ++j) {
      const int id = hd.id(j - 1);
      const uint32_t page = (uint32_t)id / (uint32_t)L.KC, slot = (uint32_t)id % (uint32_t)L.KC;
      cb[j] = (id < 0 || (long)page >= L.nb) ? -1L : (long)page * L.stride + L.o_data + (long)slot * L.cb;
    }
    const int tpc = 2 * L.BS / bits;  // tokens per chunk
    const long rowb = 2L * L.H * L.D * bits / 8;
    const long within = (long)h * (L.D * bits / 8) + c * (bits / 2);
#pragma unroll
    for (int u = 0; u < TPT; ++u) {
      const int pos = grp * KG + r * TPT + u;
      const int j = pos / tpc;
      const long base = j == 0 ? cb[0] : (j == 1 ? cb[1] : (j == 2 ? cb[2] : cb[3]));
      if (base >= 0) {
        uint32_t q[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = quant_code(x[u][e], mi[e], sc[e], bits);
        store_codes4(a.pages + base + (pos % tpc) * rowb + within, pack4(q, bits), bits);
      }
    }
  }
  // Residual K of the deferred rows whose position this thread holds.
  if (act) {
    for (int d = 0; d < def.n; ++d) {
      if (def.row[d] / TPT != r) continue;
      float k[4];
      ld_n<4>(a.key, a.kv_dtype, def.t[d] * a.k_s0 + h * a.k_s1 + 4 * c, k);
      st_n<4>(a.res.ptr, a.res.dtype, rs_raw * a.res.s0 + (long)def.row[d] * a.res.s1 + h * a.res.s2 + 4 * c, k);
    }
  }
}

template <int DT>
__device__ __forceinline__ void fin_split_t(const StepArgs& s, const FinHead& fh, int part, const Deferred& def,
                                            const int64_t* grow) {
  switch (s.w.L.KG) {
    case 8: fin_split<DT, 2>(s, fh, part, def, grow); break;
    case 16: fin_split<DT, 4>(s, fh, part, def, grow); break;
    case 32: fin_split<DT, 8>(s, fh, part, def, grow); break;
    default: fin_split<DT, 16>(s, fh, part, def, grow); break;  // 64 (the host picks this path for 8 to 64)
  }
}

// Token row t of a fused step: round trip 1 takes the row's plan and values, the
// device count and the fin rows' residual slots; the residual vote runs with the
// row's second round trip (page header, sealed stats) in flight.
__device__ __forceinline__ void step_token_row(const StepArgs& s, long t) {
  const WriteTokArgs& a = s.w;
  const int w = 3 + a.L.KG;
  const long count = *s.fin_count;
  const long rslot = a.tok[a.tok_s0 + t];
  const long r0 = (long)threadIdx.x < s.fin_grid ? s.fin[threadIdx.x * w + 2] : -1;
  auto res_here = [&]() {
    bool hit = false;
    if (rslot >= 0) {
      hit = (long)threadIdx.x < count && r0 == rslot;
      for (long f = threadIdx.x + kThreads; f < s.fin_grid; f += kThreads) {
        const long rf = s.fin[f * w + 2];
        hit = hit || (f < count && rf == rslot);
      }
    }
    return !__syncthreads_or(hit);
  };
  write_token_row(a, t, res_here);
}

__global__ __launch_bounds__(kThreads) void write_step_kernel(StepArgs s) {
  extern __shared__ uint4 step_lds[];  // fin_staged's group values (dynamic: k_group * kThreads * 8 or 16 bytes)
  __shared__ Deferred def;
  __shared__ int64_t grow[kMaxDeferred];  // the fin row's token row per position
  const long fin_wgs = s.fin_parts > 0 ? s.fin_grid * s.fin_parts : s.fin_grid;
  if ((long)blockIdx.x < fin_wgs) {
    if (s.fin_parts > 0) {  // split fin rows: staged dtype, k_group 8 to 64
      const long f = blockIdx.x / s.fin_parts;
      const int part = (int)(blockIdx.x % s.fin_parts);
      FinHead fh;
      if (!fin_prologue(s, f, def, grow, &fh)) return;
      if (s.staged == ECHOKV_F16) fin_split_t<ECHOKV_F16>(s, fh, part, def, grow);
      else if (s.staged == ECHOKV_BF16) fin_split_t<ECHOKV_BF16>(s, fh, part, def, grow);
      else fin_split_t<ECHOKV_F32>(s, fh, part, def, grow);
      return;
    }
    const long f = blockIdx.x;
    const bool staged = s.staged >= 0;
    if (!fin_prologue(s, f, def, staged ? grow : nullptr)) return;
    if (s.staged == ECHOKV_F16) {
      fin_staged<ECHOKV_F16>(s, f, (uint2*)step_lds, def, grow);
    } else if (s.staged == ECHOKV_BF16) {
      fin_staged<ECHOKV_BF16>(s, f, (uint2*)step_lds, def, grow);
    } else if (s.staged == ECHOKV_F32) {
      fin_staged<ECHOKV_F32>(s, f, step_lds, def, grow);
    } else {
      const WriteTokArgs& a = s.w;
      const FinArgs fa{a.L, a.pages, a.key, a.k_s0, a.k_s1, a.kv_dtype, s.fin, s.fin_count, a.res};
      finalize_row(fa, f, &a, &def);
    }
    return;
  }
  step_token_row(s, (long)blockIdx.x - fin_wgs);
}

// ---------------------------------------------------------------------------
// seal (echokv_vllm/tiered_cache.py:379-394): ev rows (slot, block, group, fill, bits, mask)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void seal_kernel(SealArgs a) {
  const Lay& L = a.L;
  const int64_t* e = a.ev + blockIdx.x * 6;
  const long slot = e[0], blk = e[1];
  const int grp = (int)e[2], fill = (int)e[3], bits = tier_of((uint32_t)e[4]);
  if (fill <= 0 || slot < 0 || slot >= a.res.rows || blk < 0 || blk >= L.nb || grp < 0 || grp >= L.BS / L.KG)
    return;
  const int n = fill < L.KG ? fill : L.KG;
  const int quads = L.D / 4;
  for (int i = threadIdx.x; i < L.H * quads; i += kThreads) {
    const int h = i / quads, c = i % quads;
    auto fetch = [&](int p, float x[4]) {
      ld4(a.res.ptr, a.res.dtype, slot * a.res.s0 + (long)p * a.res.s1 + h * a.res.s2 + 4 * c, x);
    };
    quantize_k_group(L, a.pages, blk, grp, grp * L.KG, n, bits, h, c, fetch);
  }
  if (threadIdx.x == 0) a.pages[blk * L.stride + 1] = (uint8_t)e[5];
}

// ---------------------------------------------------------------------------
// store_blocks: whole-block requantization from float32 K/V (demotion,
// echokv_vllm/tiered_cache.py:322-340). K per channel over each K group, V per
// token; the tag byte becomes `bits`.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void store_blocks_kernel(StoreBlkArgs a) {
  const Lay& L = a.L;
  const long b = blockIdx.x;
  const long blk = a.blocks[b];
  if (blk < 0 || blk >= L.nb) return;
  const int bits = a.bits;
  if (threadIdx.x == 0) a.pages[blk * L.stride] = (uint8_t)bits;
  const int quads = L.D / 4;
  const long rowsz = (long)L.H * L.D;
  const float* kb = a.k + b * L.BS * rowsz;
  const float* vb = a.v + b * L.BS * rowsz;
  for (int grp = 0; grp < L.BS / L.KG; ++grp) {
    for (int i = threadIdx.x; i < L.H * quads; i += kThreads) {
      const int h = i / quads, c = i % quads;
      auto fetch = [&](int p, float x[4]) {
        const float* src = kb + (long)(grp * L.KG + p) * rowsz + h * L.D + 4 * c;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = src[e];
      };
      quantize_k_group(L, a.pages, blk, grp, grp * L.KG, L.KG, bits, h, c, fetch);
    }
  }
  const int side = L.H * L.D * bits / 8;
  const int items = L.H * quads;
  for (int off = 0; off < L.BS; ++off) {
    const long rb = row_base(a.pages, L, blk, off, bits);
    for (int base = 0; base < items; base += kThreads) {
      const int i = base + (int)threadIdx.x;
      const bool act = i < items;
      const int h = act ? i / quads : 0, c = act ? i % quads : 0;
      float x[4] = {0.f, 0.f, 0.f, 0.f};
      if (act) {
        const float* src = vb + (long)off * rowsz + h * L.D + 4 * c;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = src[e];
      }
      float mn = fminf(fminf(x[0], x[1]), fminf(x[2], x[3]));
      float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      if (v_segments(L)) seg_minmax(mn, mx, L.VG / 4);  // uniform branch
      if (!act || rb < 0) continue;
      const float* vrow = vb + (long)off * rowsz + h * L.D;
      store_v4(L, a.pages, blk, rb + side, off, h, c, x, bits, mn, mx, [&](int ch) { return vrow[ch]; });
    }
  }
}

// ---------------------------------------------------------------------------
// Dequantization of one token (head h, channels 4c..4c+3): K from the residual
// when it is the block's open group, else codes x per-channel stats; V codes x
// per-token stats. `bits` is already resolved by the caller.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void dequant_token4(const Lay& L, const uint8_t* pages, const int64_t* block_res,
                                               const int64_t* res_group, const Res& res, long blk, int off,
                                               int bits, int h, int c, float k[4], float v[4]) {
  const long rb = row_base(pages, L, blk, off, bits);
  const int G = L.D / L.VG;
  if (rb < 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) k[e] = v[e] = 0.f;
    return;
  }
  const long hb = (long)h * (L.D * bits / 8) + c * (bits / 2);
  const uint32_t vc = load_codes4(pages + rb + L.H * L.D * bits / 8 + hb, bits);
  const long ve = ((long)off * L.H + h) * G;
#pragma unroll
  for (int e = 0; e < 4; ++e) {  // channel 4c + e's V group (one for every e unless VG is not a lane segment)
    const long vg = ve + (v_segments(L) ? 4 * c : 4 * c + e) / L.VG;
    const float vs = (float)*f16p(pages, blk * L.stride + L.o_vs + 2 * vg);
    const float vm = (float)*f16p(pages, blk * L.stride + L.o_vm + 2 * vg);
    v[e] = code_at(vc, e, bits) * vs + vm;
  }
  const long rs = block_res[blk];
  const int grp = off / L.KG;
  if (rs >= 0 && rs < res.rows && res_group[rs] == grp) {
    ld4(res.ptr, res.dtype, rs * res.s0 + (long)(off % L.KG) * res.s1 + h * res.s2 + 4 * c, k);
    return;
  }
  const uint32_t kc = load_codes4(pages + rb + hb, bits);
  const long se = ((long)grp * L.H + h) * L.D + 4 * c;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float ks = (float)*f16p(pages, blk * L.stride + L.o_ks + 2 * (se + e));
    const float km = (float)*f16p(pages, blk * L.stride + L.o_km + 2 * (se + e));
    k[e] = code_at(kc, e, bits) * ks + km;
  }
}

// ---------------------------------------------------------------------------
// Own-group attention of a prefill chunk, merged into the rest. A query at
// position p attends to its own K group [p & ~(KG-1), p] with the keys at full
// precision -- this step's key rows where the chunk holds them (positions >= c0),
// the cache before that -- and V from the cache, as decode saw those keys while
// the group was open; the prefill kernels attended to every key before the group
// (part_o, fp32, normalized, and its log2-domain log-sum-exp). The two merge by
// log-sum-exp into `out`. One workgroup per (query token, KV head).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void own_group_kernel(OwnGroupArgs a) {
  const Lay& L = a.L;
  const int32_t* rw = a.rows + (long)blockIdx.x * 4;
  const long q_row = rw[0];
  const int p = rw[1], c0 = rw[2];
  const long bt_row = rw[3];
  const int h = blockIdx.y;
  const int gs = p & ~(L.KG - 1);
  // A query closing its group saw the whole prefix from the cache (the prefill
  // kernels took it): no own part.
  const int nk = ((p + 1) & (L.KG - 1)) ? p - gs + 1 : 0;  // <= KG <= kOgMaxKeys
  const int quads = L.D / 4;
  __shared__ float ks[kOgMaxKeys][kOgMaxD], vs[kOgMaxKeys][kOgMaxD], qs[kOgMaxGqa][kOgMaxD];
  __shared__ float sc[kOgMaxGqa][kOgMaxKeys];
  // K and V of the group's keys (4 channels per item).
  for (int i = threadIdx.x; i < nk * quads; i += kThreads) {
    const int j = i / quads, c = i % quads;
    const int pos = gs + j;
    const long blk = a.bt[bt_row * a.bt_s0 + pos / L.BS];
    float k[4] = {0.f, 0.f, 0.f, 0.f}, v[4] = {0.f, 0.f, 0.f, 0.f};
    if (blk >= 0 && blk < L.nb) {
      const int bits = tier_of(a.pages[blk * L.stride]);
      dequant_token4(L, a.pages, a.block_res, a.res_group, a.res, blk, pos % L.BS, bits, h, c, k, v);
    }
    if (pos >= c0) ld4(a.key, a.k_dtype, (q_row - (p - pos)) * a.k_s0 + (long)h * a.k_s1 + 4 * c, k);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ks[j][4 * c + e] = k[e];
      vs[j][4 * c + e] = v[e];
    }
  }
  for (int i = threadIdx.x; i < a.gqa * L.D; i += kThreads) {
    const int g = i / L.D, d = i % L.D;
    qs[g][d] = ld(a.q, a.q_dtype, q_row * a.q_s0 + (long)(h * a.gqa + g) * a.q_s1 + d);
  }
  __syncthreads();
  // Scores (log2 units).
  for (int i = threadIdx.x; i < a.gqa * nk; i += kThreads) {
    const int g = i / nk, j = i % nk;
    float x = 0.f;
    for (int d = 0; d < L.D; ++d) x = __builtin_fmaf(qs[g][d], ks[j][d], x);
    sc[g][j] = x * a.scale_log2;
  }
  __syncthreads();
  // Softmax over the group per query head, then the merge with the earlier keys.
  for (int i = threadIdx.x; i < a.gqa * L.D; i += kThreads) {
    const int g = i / L.D, d = i % L.D;
    float m = -__builtin_inff();
    for (int j = 0; j < nk; ++j) m = fmaxf(m, sc[g][j]);
    float l = 0.f, o = 0.f;
    for (int j = 0; j < nk; ++j) {
      const float w = __builtin_amdgcn_exp2f(sc[g][j] - m);
      l += w;
      o = __builtin_fmaf(w, vs[j][d], o);
    }
    const long qh = (long)h * a.gqa + g;
    const float lse_b = nk ? m + __log2f(l) : -__builtin_inff();
    const float lse_a = a.lse[q_row * a.hq + qh];
    const float o_a = a.part[q_row * a.p_s0 + qh * a.p_s1 + d];
    const float mm = fmaxf(lse_a, lse_b);
    const float wa = lse_a == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(lse_a - mm);
    const float wb = nk ? __builtin_amdgcn_exp2f(lse_b - mm) : 0.f;
    st(a.out, a.out_dtype, q_row * a.o_s0 + qh * a.o_s1 + d, nk ? (wa * o_a + wb * (o / l)) / (wa + wb) : o_a);
  }
}

// gather (echokv_vllm/tiered_cache.py:451-478): never-opened blocks read as zeros.

__global__ __launch_bounds__(kThreads) void gather_kernel(GatherArgs a) {
  const Lay& L = a.L;
  const long i = blockIdx.x;
  const long blk = a.blk[i];
  const int off = (int)a.off[i];
  const int quads = L.D / 4;
  const long ob = i * (long)L.H * L.D;
  const bool ok = blk >= 0 && blk < L.nb && off >= 0 && off < L.BS;
  const uint32_t tag = ok ? a.pages[blk * L.stride] : 0u;
  const bool opened = tag == 2u || tag == 4u || tag == 8u;
  for (int it = threadIdx.x; it < L.H * quads; it += kThreads) {
    const int h = it / quads, c = it % quads;
    float k[4] = {0.f, 0.f, 0.f, 0.f}, v[4] = {0.f, 0.f, 0.f, 0.f};
    if (opened) dequant_token4(L, a.pages, a.block_res, a.res_group, a.res, blk, off, (int)tag, h, c, k, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a.k_out[ob + h * L.D + 4 * c + e] = k[e];
      a.v_out[ob + h * L.D + 4 * c + e] = v[e];
    }
  }
}

// dequant_dense (echokv_vllm/kernels/prefill.py:90-115, 330-369): work rows
// (block-table row, block index, dense row of the block start, ctx).

__global__ __launch_bounds__(kThreads) void dequant_dense_kernel(DenseArgs a) {
  const Lay& L = a.L;
  const int32_t* w = a.work + blockIdx.x * 4;
  const long req = w[0];
  const int bi = w[1];
  const long row0 = w[2];
  const int ctx = w[3];
  const long blk = a.bt[req * a.bt_s0 + bi];
  if (blk < 0 || blk >= L.nb) return;
  const int bits = tier_of(a.pages[blk * L.stride]);
  const int quads = L.D / 4;
  int n = ctx - bi * L.BS;
  n = n < L.BS ? n : L.BS;
  const int items = n * L.H * quads;
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int t = it / (L.H * quads);
    const int r = it % (L.H * quads);
    const int h = r / quads, c = r % quads;
    float k[4], v[4];
    dequant_token4(L, a.pages, a.block_res, a.res_group, a.res, blk, t, bits, h, c, k, v);
    const long o = (row0 + t) * a.o_s0 + h * a.o_s1 + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      st(a.k_out, a.out_dtype, o + e, k[e]);
      st(a.v_out, a.out_dtype, o + e, v[e]);
    }
  }
}

}  // namespace ek

// ---------------------------------------------------------------------------
// Launchers (called from abi.hip)
// ---------------------------------------------------------------------------
namespace ek {

hipError_t launch_write_tokens(const WriteTokArgs& a, long n_rows, hipStream_t s) {
  hipLaunchKernelGGL(write_tokens_kernel, dim3((unsigned)n_rows), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_finalize_k(const FinArgs& a, long rows, hipStream_t s) {
  hipLaunchKernelGGL(finalize_k_kernel, dim3((unsigned)rows), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_write_step(const StepArgs& a, hipStream_t s) {
  const size_t lds = a.staged < 0 || a.fin_parts > 0 ? 0 : step_staged_lds(a.w.L.KG, a.staged);
  const long fin_wgs = a.fin_parts > 0 ? a.fin_grid * a.fin_parts : a.fin_grid;
  hipLaunchKernelGGL(write_step_kernel, dim3((unsigned)(fin_wgs + a.n_rows)), dim3(kThreads), lds, s, a);
  return hipGetLastError();
}
// Page headers of a step's freshly opened blocks in every layer, one launch: layer
// l's 16 header bytes of block ids[i] are hdr[l * n + i], at page_bases[l] +
// ids[i] * page_stride. Four 32-bit stores (page bases need only 4-byte alignment).
__global__ __launch_bounds__(kThreads) void write_headers_kernel(const uint64_t* page_bases, long page_stride,
                                                                  const int64_t* ids, const uint32_t* hdr,
                                                                  int n_layers, long n) {
  const long i = (long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n_layers * n) return;
  const long l = i / n, b = i - l * n;
  uint32_t* dst = (uint32_t*)(page_bases[l] + (uint64_t)(ids[b] * page_stride));
  const uint32_t* src = hdr + 4 * i;
#pragma unroll
  for (int e = 0; e < 4; ++e) dst[e] = src[e];
}

hipError_t launch_write_headers(const uint64_t* page_bases, long page_stride, const int64_t* ids,
                                const uint32_t* hdr, int n_layers, long n, hipStream_t s) {
  const long total = n_layers * n;
  hipLaunchKernelGGL(write_headers_kernel, dim3((unsigned)((total + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                     page_bases, page_stride, ids, hdr, n_layers, n);
  return hipGetLastError();
}

hipError_t launch_seal(const SealArgs& a, long n, hipStream_t s) {
  hipLaunchKernelGGL(seal_kernel, dim3((unsigned)n), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_store_blocks(const StoreBlkArgs& a, long n, hipStream_t s) {
  hipLaunchKernelGGL(store_blocks_kernel, dim3((unsigned)n), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_gather(const GatherArgs& a, long n, hipStream_t s) {
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)n), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_own_group(const OwnGroupArgs& a, long n, hipStream_t s) {
  hipLaunchKernelGGL(own_group_kernel, dim3((unsigned)n, (unsigned)a.L.H), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_dequant_dense(const DenseArgs& a, long n, hipStream_t s) {
  hipLaunchKernelGGL(dequant_dense_kernel, dim3((unsigned)n), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace ek
