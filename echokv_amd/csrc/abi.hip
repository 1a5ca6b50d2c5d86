// extern "C" entry points of libechokv.so (declared in include/echokv.h):
// argument checks on the host, then asynchronous kernel launches on the
// caller's stream. Nothing here allocates, synchronizes or touches device data.
#include "args.h"

namespace {

bool lay_ok(const echokv_layout* L) {
  if (!L) return false;
  const int H = L->num_kv_heads, D = L->head_size, BS = L->block_size, KG = L->k_group, VG = L->v_group;
  if (H <= 0 || D <= 0 || BS <= 0 || KG <= 0 || VG <= 0 || L->chunks_per_page <= 0 || L->num_blocks <= 0) return false;
  if (D % 4 || D % VG || BS % 16 || BS % KG || VG > 256) return false;
  if (L->page_stride % 16 || L->chunk_bytes != (int64_t)BS * H * D / 2) return false;
  return true;
}

ek::Lay to_lay(const echokv_layout* L) {
  ek::Lay d;
  d.H = L->num_kv_heads;
  d.D = L->head_size;
  d.BS = L->block_size;
  d.KG = L->k_group;
  d.VG = L->v_group;
  d.KC = L->chunks_per_page;
  d.nb = L->num_blocks;
  d.stride = L->page_stride;
  d.o_vs = L->o_v_scale;
  d.o_vm = L->o_v_min;
  d.o_ks = L->o_k_scale;
  d.o_km = L->o_k_min;
  d.o_data = L->o_data;
  d.cb = L->chunk_bytes;
  return d;
}

bool dtype_ok(int dt) { return dt == ECHOKV_F32 || dt == ECHOKV_F16 || dt == ECHOKV_BF16; }

bool res_ok(const echokv_residual* r) { return r && r->ptr && dtype_ok(r->dtype) && r->rows >= 1; }

ek::Res to_res(const echokv_residual* r) {
  ek::Res d;
  d.ptr = r->ptr;
  d.dtype = r->dtype;
  d.rows = r->rows;
  d.s0 = r->s0;
  d.s1 = r->s1;
  d.s2 = r->s2;
  return d;
}

int launched(hipError_t e) { return e == hipSuccess ? ECHOKV_OK : ECHOKV_ELAUNCH; }

}  // namespace

extern "C" {

const char* echokv_error_string(int code) {
  switch (code) {
    case ECHOKV_OK: return "ok";
    case ECHOKV_EINVAL: return "invalid argument (null pointer, count or stride)";
    case ECHOKV_ESHAPE: return "layout or head shape not supported by this build";
    case ECHOKV_EDTYPE: return "unsupported dtype";
    case ECHOKV_ELAUNCH: return "kernel launch failed";
    case ECHOKV_ETOOBIG: return "the request needs more than the library's static scratch buffer";
    default: return "unknown error";
  }
}

int echokv_write_tokens(const echokv_layout* L, uint8_t* pages, const void* key, int64_t k_s0, int64_t k_s1,
                        const void* value, int64_t v_s0, int64_t v_s1, int32_t kv_dtype, const int64_t* tok,
                        int64_t tok_s0, int64_t n_rows, const echokv_residual* res, float* kref, int64_t kref_s0,
                        int64_t kref_s1, echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (!dtype_ok(kv_dtype)) return ECHOKV_EDTYPE;
  if (n_rows < 0 || tok_s0 < n_rows || !res_ok(res)) return ECHOKV_EINVAL;
  if (n_rows == 0) return ECHOKV_OK;
  if (!pages || !key || !value || !tok) return ECHOKV_EINVAL;
  ek::WriteTokArgs a{to_lay(L), pages, key, k_s0, k_s1, value, v_s0, v_s1, kv_dtype, tok, tok_s0, to_res(res),
                     kref, kref_s0, kref_s1};
  return launched(ek::launch_write_tokens(a, n_rows, (hipStream_t)stream));
}

int echokv_finalize_k(const echokv_layout* L, uint8_t* pages, const void* key, int64_t k_s0, int64_t k_s1,
                      int32_t kv_dtype, const int64_t* fin, const int64_t* fin_count, int64_t grid_rows,
                      const echokv_residual* res, echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (!dtype_ok(kv_dtype)) return ECHOKV_EDTYPE;
  if (grid_rows < 0 || !res_ok(res)) return ECHOKV_EINVAL;
  if (grid_rows == 0) return ECHOKV_OK;
  if (!pages || !key || !fin || !fin_count) return ECHOKV_EINVAL;
  ek::FinArgs a{to_lay(L), pages, key, k_s0, k_s1, kv_dtype, fin, fin_count, to_res(res)};
  return launched(ek::launch_finalize_k(a, grid_rows, (hipStream_t)stream));
}

int echokv_write_step(const echokv_layout* L, uint8_t* pages, const void* key, int64_t k_s0, int64_t k_s1,
                      const void* value, int64_t v_s0, int64_t v_s1, int32_t kv_dtype, const int64_t* tok,
                      int64_t tok_s0, int64_t n_rows, const int64_t* fin, const int64_t* fin_count, int64_t fin_grid,
                      const echokv_residual* res, float* kref, int64_t kref_s0, int64_t kref_s1,
                      echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (L->k_group > ek::kMaxDeferred) return ECHOKV_ESHAPE;
  if (!dtype_ok(kv_dtype)) return ECHOKV_EDTYPE;
  if (n_rows < 0 || fin_grid < 0 || tok_s0 < n_rows || !res_ok(res)) return ECHOKV_EINVAL;
  if (n_rows + fin_grid == 0) return ECHOKV_OK;
  if (!pages || !key || !fin_count || (n_rows && (!value || !tok)) || (fin_grid && !fin)) return ECHOKV_EINVAL;
  // Fin rows read their group with one vector load per four channels when key and
  // residual share a dtype and every four-channel run is aligned for it. Such rows
  // are split over workgroups of 64 (head, quad) items, a group over 4 lanes per
  // item, for k_group 8 to 64; other k_groups stage the group in LDS when it fits.
  const int KG = L->k_group;
  const uintptr_t al = kv_dtype == ECHOKV_F32 ? 16 : 8;
  const bool vec = kv_dtype == res->dtype && (uintptr_t)key % al == 0 && (uintptr_t)res->ptr % al == 0 &&
                   k_s0 % 4 == 0 && k_s1 % 4 == 0 && res->s0 % 4 == 0 && res->s1 % 4 == 0 && res->s2 % 4 == 0;
  const int items = L->num_kv_heads * (L->head_size / 4);
  const int parts = vec && KG >= 8 && KG <= 64 && !(KG & (KG - 1)) ? (items + 63) / 64 : 0;
  if (parts > 0 && fin_grid > INT32_MAX / parts) return ECHOKV_EINVAL;
  const int staged =
      vec && (parts > 0 || ek::step_staged_lds(KG, kv_dtype) <= ek::kStepStagedMaxLds) ? kv_dtype : -1;
  ek::StepArgs a{ek::WriteTokArgs{to_lay(L), pages, key, k_s0, k_s1, value, v_s0, v_s1, kv_dtype, tok, tok_s0,
                                  to_res(res), kref, kref_s0, kref_s1},
                 fin, fin_count, fin_grid, n_rows, staged, parts};
  return launched(ek::launch_write_step(a, (hipStream_t)stream));
}

int echokv_seal_groups(const echokv_layout* L, uint8_t* pages, const int64_t* ev, int64_t n,
                       const echokv_residual* res, echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (n < 0 || !res_ok(res)) return ECHOKV_EINVAL;
  if (n == 0) return ECHOKV_OK;
  if (!pages || !ev) return ECHOKV_EINVAL;
  ek::SealArgs a{to_lay(L), pages, ev, to_res(res)};
  return launched(ek::launch_seal(a, n, (hipStream_t)stream));
}

int echokv_gather(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res, const int64_t* res_group,
                  const echokv_residual* res, const int64_t* blk, const int64_t* off, int64_t n, float* k_out,
                  float* v_out, echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (n < 0 || !res_ok(res)) return ECHOKV_EINVAL;
  if (n == 0) return ECHOKV_OK;
  if (!pages || !block_res || !res_group || !blk || !off || !k_out || !v_out) return ECHOKV_EINVAL;
  ek::GatherArgs a{to_lay(L), pages, block_res, res_group, to_res(res), blk, off, k_out, v_out};
  return launched(ek::launch_gather(a, n, (hipStream_t)stream));
}

int echokv_write_headers(const uint64_t* page_bases, int32_t n_layers, int64_t page_stride, const int64_t* ids,
                         int64_t n, const uint8_t* headers, echokv_stream_t stream) {
  if (n_layers < 0 || n < 0 || page_stride < 16 || page_stride % 4) return ECHOKV_EINVAL;
  if (n_layers == 0 || n == 0) return ECHOKV_OK;
  if ((int64_t)n_layers * n > INT32_MAX || ((uintptr_t)headers & 3)) return ECHOKV_EINVAL;
  if (!page_bases || !ids || !headers) return ECHOKV_EINVAL;
  return launched(ek::launch_write_headers(page_bases, page_stride, ids, (const uint32_t*)headers, n_layers, n,
                                           (hipStream_t)stream));
}

int echokv_store_blocks(const echokv_layout* L, uint8_t* pages, const int64_t* blocks, int64_t n, const float* k,
                        const float* v, int32_t bits, echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (n < 0 || (bits != 2 && bits != 4 && bits != 8)) return ECHOKV_EINVAL;
  if (n == 0) return ECHOKV_OK;
  if (!pages || !blocks || !k || !v) return ECHOKV_EINVAL;
  ek::StoreBlkArgs a{to_lay(L), pages, blocks, k, v, bits};
  return launched(ek::launch_store_blocks(a, n, (hipStream_t)stream));
}

}  // extern "C"

namespace {

// The MFMA decode kernels take: D 64 or 128 with at least D/16 channels per V
// group, or D 256 as half-heads of 128 (V groups of 8 to 128 channels: each
// inside one half), 16-token tiles inside one K group (one k_scale / k_min row per
// tile), power-of-two block size and K group, <= 4 chunks per page. Any other
// layout takes decode_any.
bool decode_mfma(const echokv_layout* L) {
  const bool pow2 = !(L->block_size & (L->block_size - 1)) && !(L->k_group & (L->k_group - 1));
  const int D = L->head_size, VG = L->v_group;
  const bool heads = D == 256 ? VG <= 128 && VG % 8 == 0 : (D == 64 || D == 128) && VG % (D / 16) == 0;
  return heads && L->k_group >= 16 && pow2 && L->chunks_per_page <= 4 &&
         L->num_blocks * L->chunks_per_page < (1LL << 24);
}

// The layout the MFMA kernels are given: head size 256 as 2H half-heads of 128
// channels (DecodeArgs::pair; the same page bytes), any other as it is.
void decode_view(const echokv_layout* L, ek::DecodeArgs& a) {
  a.L = to_lay(L);
  a.pair = 0;
  if (L->head_size == 256 && decode_mfma(L)) {
    a.L.H = 2 * L->num_kv_heads;
    a.L.D = L->head_size / 2;
    a.pair = 1;
  }
}

// Whether the MFMA decode folds the V scale into the P operand (DecodeArgs::ps): the
// first pass's query heads times the kernel head's V groups fill at most the 16
// MFMA columns (every later pass has as many query heads or fewer).
// 2: two tiles per step (the INT8 kernel), for 4 query heads x 4 V groups at head
// size 128.
int decode_ps(const ek::DecodeArgs& a, int gqa) {
  const int G = a.L.D / a.L.VG, gs = gqa < 16 ? gqa : 16;
  if (G == 4 && gs == 4 && a.L.D == 128 && !a.pair) return 2;
  return G >= 1 && G <= 4 && gs * G <= 16 ? 1 : 0;
}

// echokv_decode and echokv_decode_static: the checks, then decode + merge with
// the given workspaces, or (static_scratch) with the library's static scratch.
int decode_run(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res, const int64_t* res_group,
               const echokv_residual* res, const void* query, int64_t q_s0, int64_t q_s1, int32_t q_dtype,
               int32_t num_q_heads, const int64_t* q_rows, const int32_t* block_table, int64_t bt_s0,
               const int64_t* bt_rows, const int64_t* seq_lens, int64_t num_seqs, float softmax_scale,
               int32_t num_splits, int32_t blocks_per_split, int32_t tier, const int32_t* tier_mask, int32_t flags,
               float* acc, float* ml, bool static_scratch, void* out, int64_t o_s0, int64_t o_s1, int32_t out_dtype,
               echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  const bool mfma = decode_mfma(L);
  if (!mfma && L->head_size > ek::kMaxAnyD) return ECHOKV_ESHAPE;
  if (num_q_heads <= 0 || num_q_heads % L->num_kv_heads) return ECHOKV_ESHAPE;
  const int gqa = num_q_heads / L->num_kv_heads;
  if (!dtype_ok(q_dtype) || !dtype_ok(out_dtype)) return ECHOKV_EDTYPE;
  if (num_seqs < 0 || num_splits <= 0 || blocks_per_split <= 0 || !res_ok(res)) return ECHOKV_EINVAL;
  if (tier != 2 && tier != 4 && tier != 8) return ECHOKV_EINVAL;
  if (flags & ~ECHOKV_DECODE_BATCH_INVARIANT) return ECHOKV_EINVAL;
  if (tier_mask && !(flags & ECHOKV_DECODE_BATCH_INVARIANT)) return ECHOKV_EINVAL;  // tier passes: split schedule
  if (num_seqs == 0) return ECHOKV_OK;
  if (!pages || !block_res || !res_group || !query || !block_table || !seq_lens || !out) return ECHOKV_EINVAL;
  if (!static_scratch && (!acc || !ml)) return ECHOKV_EINVAL;
  ek::DecodeArgs a;
  decode_view(L, a);
  a.pages = pages;
  a.block_res = block_res;
  a.res_group = res_group;
  a.res = to_res(res);
  a.q = query;
  a.q_s0 = q_s0;
  a.q_s1 = q_s1;
  a.q_dtype = q_dtype;
  a.hq = num_q_heads;
  a.gqa = gqa;
  a.q_rows = q_rows;
  a.bt = block_table;
  a.bt_s0 = bt_s0;
  a.bt_rows = bt_rows;
  a.lens = seq_lens;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.num_splits = num_splits;
  a.bps = blocks_per_split;
  a.num_seqs = num_seqs;
  a.tier = tier;
  a.tier0 = tier;
  a.tier_mask = nullptr;
  a.bs_shift = mfma ? __builtin_ctz((unsigned)L->block_size) : 0;
  a.kg_shift = mfma ? __builtin_ctz((unsigned)L->k_group) : 0;
  a.vg_shift = __builtin_ctz((unsigned)L->v_group);
  // ceil(2^32 / KC) is exact for chunk ids < 2^24 (fractions of id / KC are multiples of 1 / KC >= 1/4).
  a.kc_mul = !mfma || L->chunks_per_page == 1
                 ? 0u
                 : (uint32_t)((0x100000000ull + L->chunks_per_page - 1) / L->chunks_per_page);
  if (!mfma && num_seqs > INT32_MAX / L->num_kv_heads / num_splits) return ECHOKV_ESHAPE;  // one workgroup each
  if (static_scratch) {
    // acc [S, Hq, splits, D] then ml [S, Hq, splits, 2], float32, in the static array.
    if (num_seqs > (1LL << 31) / num_q_heads / num_splits) return ECHOKV_ETOOBIG;
    const int64_t rows = num_seqs * num_q_heads * num_splits;
    if (rows * (L->head_size + 2) * 4 > (int64_t)ek::kDecodeScratchBytes) return ECHOKV_ETOOBIG;
    void* base = nullptr;
    if (ek::decode_scratch(&base) != hipSuccess) return ECHOKV_ELAUNCH;
    acc = (float*)base;
    ml = acc + rows * L->head_size;
  }
  a.acc = acc;
  a.ml = ml;
  a.out = out;
  a.o_s0 = o_s0;
  a.o_s1 = o_s1;
  a.out_dtype = out_dtype;
  a.ranges = 0;
  a.ps = mfma ? decode_ps(a, gqa) : 0;
  if (mfma && !(flags & ECHOKV_DECODE_BATCH_INVARIANT) && ek::decode_ranges(a, a.ranges) != hipSuccess)
    return ECHOKV_ELAUNCH;
  // A wave's MFMA columns hold 16 query heads: a larger GQA runs in passes of 16
  // query heads per KV head (each pass reads the cache again; their rows are disjoint).
  for (int g0 = 0; g0 < gqa; g0 += 16) {
    a.g0 = g0;
    a.gs = gqa - g0 < 16 ? gqa - g0 : 16;
    if (mfma && tier_mask) {
      // One launch per tier, lowest first: each runs only if the layer holds its
      // tier (read from tier_mask when it runs) and continues the partial rows the
      // one before it left.
      a.tier_mask = tier_mask;
      for (int t : {2, 4, 8}) {
        a.tier = t;
        if (ek::launch_decode(a, num_seqs, (hipStream_t)stream) != hipSuccess) return ECHOKV_ELAUNCH;
      }
      a.tier = tier;
      a.tier_mask = nullptr;
    } else {
      const hipError_t d = mfma ? ek::launch_decode(a, num_seqs, (hipStream_t)stream)
                                : ek::launch_decode_any(a, (hipStream_t)stream);
      if (d != hipSuccess) return ECHOKV_ELAUNCH;
    }
    hipError_t e;
    if (a.ranges > 0) {
      e = ek::launch_merge_balanced(a, (hipStream_t)stream);
    } else {
      ek::MergeArgs m{acc, ml, seq_lens, q_rows, out, o_s0, o_s1, out_dtype, num_q_heads, L->head_size,
                      L->block_size, num_splits, blocks_per_split, num_seqs * num_q_heads, gqa, a.g0, a.gs};
      e = mfma ? ek::launch_merge(m, num_seqs, (hipStream_t)stream) : ek::launch_merge_any(m, (hipStream_t)stream);
    }
    if (e != hipSuccess) return ECHOKV_ELAUNCH;
  }
  return ECHOKV_OK;
}

}  // namespace

extern "C" {

int echokv_decode(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res, const int64_t* res_group,
                  const echokv_residual* res, const void* query, int64_t q_s0, int64_t q_s1, int32_t q_dtype,
                  int32_t num_q_heads, const int64_t* q_rows, const int32_t* block_table, int64_t bt_s0,
                  const int64_t* bt_rows, const int64_t* seq_lens, int64_t num_seqs, float softmax_scale,
                  int32_t num_splits, int32_t blocks_per_split, int32_t tier, const int32_t* tier_mask,
                  int32_t flags, float* acc, float* ml, void* out, int64_t o_s0, int64_t o_s1, int32_t out_dtype,
                  echokv_stream_t stream) {
  return decode_run(L, pages, block_res, res_group, res, query, q_s0, q_s1, q_dtype, num_q_heads, q_rows,
                    block_table, bt_s0, bt_rows, seq_lens, num_seqs, softmax_scale, num_splits, blocks_per_split,
                    tier, tier_mask, flags, acc, ml, false, out, o_s0, o_s1, out_dtype, stream);
}

int echokv_decode_static(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                         const int64_t* res_group, const echokv_residual* res, const void* query, int64_t q_s0,
                         int64_t q_s1, int32_t q_dtype, int32_t num_q_heads, const int64_t* q_rows,
                         const int32_t* block_table, int64_t bt_s0, const int64_t* bt_rows, const int64_t* seq_lens,
                         int64_t num_seqs, float softmax_scale, int32_t num_splits, int32_t blocks_per_split,
                         int32_t tier, const int32_t* tier_mask, int32_t flags, void* out, int64_t o_s0,
                         int64_t o_s1, int32_t out_dtype, echokv_stream_t stream) {
  return decode_run(L, pages, block_res, res_group, res, query, q_s0, q_s1, q_dtype, num_q_heads, q_rows,
                    block_table, bt_s0, bt_rows, seq_lens, num_seqs, softmax_scale, num_splits, blocks_per_split,
                    tier, tier_mask, flags, nullptr, nullptr, true, out, o_s0, o_s1, out_dtype, stream);
}

int64_t echokv_decode_workspace_rows(const echokv_layout* L, int32_t num_q_heads, int32_t q_dtype,
                                     int64_t num_seqs, int32_t num_splits, int32_t flags) {
  if (!lay_ok(L) || num_q_heads <= 0 || num_q_heads % L->num_kv_heads || num_seqs < 0 || num_splits <= 0 ||
      !dtype_ok(q_dtype) || (flags & ~ECHOKV_DECODE_BATCH_INVARIANT))
    return -1;
  const int64_t split_rows = num_seqs * num_splits;
  if (!decode_mfma(L) || (flags & ECHOKV_DECODE_BATCH_INVARIANT) || num_seqs == 0) return split_rows;
  // Balanced schedule: two partial slots per range; the range count depends on the
  // tier's kernel (its occupancy), so the largest over the tiers.
  ek::DecodeArgs a;
  decode_view(L, a);
  a.q_dtype = q_dtype;
  a.num_seqs = num_seqs;
  a.num_splits = num_splits;
  a.ps = decode_ps(a, num_q_heads / L->num_kv_heads);
  int64_t rows = 0;
  for (int tier : {2, 4, 8}) {
    a.tier = tier;
    long r = 0;
    if (ek::decode_ranges(a, r) != hipSuccess) return -1;
    rows = rows > 2 * r ? rows : 2 * r;
  }
  return rows < split_rows ? rows : split_rows;
}

int echokv_prefill(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res, const int64_t* res_group,
                   const echokv_residual* res, const void* query, int64_t q_s0, int64_t q_s1, int32_t q_dtype,
                   int32_t num_q_heads, void* out, int64_t o_s0, int64_t o_s1, int32_t out_dtype,
                   const int32_t* tiles, int64_t n_tiles, int32_t tile_m, const int32_t* block_table, int64_t bt_s0,
                   float softmax_scale, int32_t own_group, float* lse, echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (num_q_heads <= 0 || num_q_heads % L->num_kv_heads) return ECHOKV_ESHAPE;
  const int gqa = num_q_heads / L->num_kv_heads;
  // The MFMA kernel: head size 64, 128 or 256, at most prefill_rows query rows
  // per tile. Any other layout (head size up to kMaxAnyD) takes the fp32 kernel.
  const int D = L->head_size;
  const bool mfma = (D == 64 || D == 128 || D == 256) && gqa <= ek::prefill_rows(D);
  if (!mfma && (D > ek::kMaxAnyD || own_group)) return ECHOKV_ESHAPE;
  if (tile_m != (mfma ? ek::prefill_tile_tokens(gqa, D) : ek::any_tile_tokens(gqa))) return ECHOKV_ESHAPE;
  if (own_group != 0 && own_group != 1) return ECHOKV_EINVAL;
  if (own_group && (L->k_group & (L->k_group - 1))) return ECHOKV_ESHAPE;
  if (!dtype_ok(q_dtype) || !dtype_ok(out_dtype)) return ECHOKV_EDTYPE;
  if (n_tiles < 0 || !res_ok(res)) return ECHOKV_EINVAL;
  if (n_tiles == 0) return ECHOKV_OK;
  if (!pages || !block_res || !res_group || !query || !out || !tiles || !block_table) return ECHOKV_EINVAL;
  ek::PrefillArgs a;
  a.L = to_lay(L);
  a.pages = pages;
  a.block_res = block_res;
  a.res_group = res_group;
  a.res = to_res(res);
  a.q = query;
  a.q_s0 = q_s0;
  a.q_s1 = q_s1;
  a.q_dtype = q_dtype;
  a.hq = num_q_heads;
  a.gqa = gqa;
  a.out = out;
  a.o_s0 = o_s0;
  a.o_s1 = o_s1;
  a.out_dtype = out_dtype;
  a.tiles = tiles;
  a.bt = block_table;
  a.bt_s0 = bt_s0;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.og_mask = own_group ? ~(L->k_group - 1) : 0;
  a.lse = lse;
  a.g0 = 0;
  a.gs = gqa;
  if (mfma) return launched(ek::launch_prefill(a, n_tiles, (hipStream_t)stream));
  if (n_tiles > INT32_MAX / L->num_kv_heads) return ECHOKV_EINVAL;
  for (int g0 = 0; g0 < gqa; g0 += 16) {  // passes of 16 query heads per KV head
    a.g0 = g0;
    a.gs = gqa - g0 < 16 ? gqa - g0 : 16;
    if (ek::launch_prefill_any(a, n_tiles, (hipStream_t)stream) != hipSuccess) return ECHOKV_ELAUNCH;
  }
  return ECHOKV_OK;
}

int64_t echokv_prefill_dense_workspace(const echokv_layout* L, int64_t n_packs) {
  if (!lay_ok(L)) return -ECHOKV_ESHAPE;
  if (L->head_size != 64 && L->head_size != 128) return -ECHOKV_ESHAPE;
  if (n_packs < 0) return -ECHOKV_EINVAL;
  return n_packs * L->num_kv_heads * ek::dense_tile_bytes(L->head_size);
}

int echokv_prefill_dense(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                         const int64_t* res_group, const echokv_residual* res, const void* query, int64_t q_s0,
                         int64_t q_s1, int32_t q_dtype, int32_t num_q_heads, void* out, int64_t o_s0, int64_t o_s1,
                         int32_t out_dtype, const int32_t* packs, int64_t n_packs, const int32_t* qtiles,
                         int64_t n_qtiles, int32_t tile_m, const int32_t* block_table, int64_t bt_s0, void* workspace,
                         int64_t workspace_bytes, float softmax_scale, int32_t own_group, float* lse,
                         echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (L->head_size != 64 && L->head_size != 128) return ECHOKV_ESHAPE;
  if (num_q_heads <= 0 || num_q_heads % L->num_kv_heads) return ECHOKV_ESHAPE;
  const int gqa = num_q_heads / L->num_kv_heads;
  if (gqa > 32 * ek::kDenseWaves || tile_m != ek::dense_tile_tokens(gqa)) return ECHOKV_ESHAPE;
  if (own_group != 0 && own_group != 1) return ECHOKV_EINVAL;
  if (own_group && (L->k_group & (L->k_group - 1))) return ECHOKV_ESHAPE;
  if (!dtype_ok(q_dtype) || !dtype_ok(out_dtype)) return ECHOKV_EDTYPE;
  if (n_packs < 0 || n_qtiles < 0 || n_qtiles > INT32_MAX / L->num_kv_heads || !res_ok(res)) return ECHOKV_EINVAL;
  if (n_qtiles == 0) return ECHOKV_OK;
  if (workspace_bytes < n_packs * L->num_kv_heads * ek::dense_tile_bytes(L->head_size)) return ECHOKV_EINVAL;
  if (!pages || !block_res || !res_group || !query || !out || !packs || !qtiles || !block_table ||
      (n_packs > 0 && !workspace))
    return ECHOKV_EINVAL;
  const hipStream_t s = (hipStream_t)stream;
  uint8_t* ws = (uint8_t*)workspace;
  if (n_packs > 0) {
    ek::PackArgs p{to_lay(L), pages, block_res, res_group, to_res(res), packs, block_table, bt_s0, ws};
    const int rc = launched(ek::launch_prefill_pack(p, n_packs, s));
    if (rc != ECHOKV_OK) return rc;
  }
  ek::FlashArgs f;
  f.ws = ws;
  f.q = query;
  f.q_s0 = q_s0;
  f.q_s1 = q_s1;
  f.q_dtype = q_dtype;
  f.out = out;
  f.o_s0 = o_s0;
  f.o_s1 = o_s1;
  f.out_dtype = out_dtype;
  f.qtiles = qtiles;
  f.n_qtiles = (int)n_qtiles;
  f.H = L->num_kv_heads;
  f.gqa = gqa;
  f.D = L->head_size;
  f.n_packs = n_packs;
  f.scale_log2 = softmax_scale * 1.4426950408889634f;
  f.og_mask = own_group ? ~(L->k_group - 1) : 0;
  f.lse = lse;
  f.hq = num_q_heads;
  return launched(ek::launch_prefill_flash(f, s));
}

int echokv_prefill_own_group(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                             const int64_t* res_group, const echokv_residual* res, const void* query, int64_t q_s0,
                             int64_t q_s1, int32_t q_dtype, int32_t num_q_heads, const void* key, int64_t k_s0,
                             int64_t k_s1, int32_t k_dtype, const int32_t* rows, int64_t n_rows,
                             const int32_t* block_table, int64_t bt_s0, const float* part, int64_t p_s0, int64_t p_s1,
                             const float* lse, void* out, int64_t o_s0, int64_t o_s1, int32_t out_dtype,
                             float softmax_scale, echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (L->head_size > ek::kOgMaxD || L->k_group > ek::kOgMaxKeys || (L->k_group & (L->k_group - 1)))
    return ECHOKV_ESHAPE;
  if (num_q_heads <= 0 || num_q_heads % L->num_kv_heads || num_q_heads / L->num_kv_heads > ek::kOgMaxGqa)
    return ECHOKV_ESHAPE;
  if (!dtype_ok(q_dtype) || !dtype_ok(k_dtype) || !dtype_ok(out_dtype)) return ECHOKV_EDTYPE;
  if (n_rows < 0 || !res_ok(res)) return ECHOKV_EINVAL;
  if (n_rows == 0) return ECHOKV_OK;
  if (!pages || !block_res || !res_group || !query || !key || !rows || !block_table || !part || !lse || !out)
    return ECHOKV_EINVAL;
  ek::OwnGroupArgs a;
  a.L = to_lay(L);
  a.pages = pages;
  a.block_res = block_res;
  a.res_group = res_group;
  a.res = to_res(res);
  a.q = query;
  a.q_s0 = q_s0;
  a.q_s1 = q_s1;
  a.q_dtype = q_dtype;
  a.hq = num_q_heads;
  a.gqa = num_q_heads / L->num_kv_heads;
  a.key = key;
  a.k_s0 = k_s0;
  a.k_s1 = k_s1;
  a.k_dtype = k_dtype;
  a.rows = rows;
  a.bt = block_table;
  a.bt_s0 = bt_s0;
  a.part = part;
  a.p_s0 = p_s0;
  a.p_s1 = p_s1;
  a.lse = lse;
  a.out = out;
  a.o_s0 = o_s0;
  a.o_s1 = o_s1;
  a.out_dtype = out_dtype;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  return launched(ek::launch_own_group(a, n_rows, (hipStream_t)stream));
}

int echokv_dequant_dense(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                         const int64_t* res_group, const echokv_residual* res, const int32_t* work, int64_t n_work,
                         const int32_t* block_table, int64_t bt_s0, void* k_out, void* v_out, int64_t o_s0,
                         int64_t o_s1, int32_t out_dtype, echokv_stream_t stream) {
  if (!lay_ok(L)) return ECHOKV_ESHAPE;
  if (!dtype_ok(out_dtype)) return ECHOKV_EDTYPE;
  if (n_work < 0 || !res_ok(res)) return ECHOKV_EINVAL;
  if (n_work == 0) return ECHOKV_OK;
  if (!pages || !block_res || !res_group || !work || !block_table || !k_out || !v_out) return ECHOKV_EINVAL;
  ek::DenseArgs a{to_lay(L), pages, block_res, res_group, to_res(res), work, block_table, bt_s0,
                  k_out, v_out, o_s0, o_s1, out_dtype};
  return launched(ek::launch_dequant_dense(a, n_work, (hipStream_t)stream));
}

int echokv_canary_kl(const void* query, int32_t q_dtype, int64_t q_sl, int64_t q_s0, int64_t q_s1, const float* kref,
                     int64_t k_sl, int64_t k_s0, int64_t k_s1, int32_t num_layers, int32_t nq, int32_t num_q_heads,
                     int32_t num_kv_heads, int32_t head_size, int32_t window, int32_t nbits, int32_t bits_packed,
                     int32_t k_group, float softmax_scale, float* partial, float* out, echokv_stream_t stream) {
  if (!dtype_ok(q_dtype)) return ECHOKV_EDTYPE;
  if (num_layers < 0 || nq < 1 || num_kv_heads < 1 || num_q_heads < 1 || num_q_heads % num_kv_heads || k_group < 1)
    return ECHOKV_EINVAL;
  if (nbits < 1 || nbits > ek::kCanaryMaxTiers) return ECHOKV_EINVAL;
  for (int t = 0; t < nbits; ++t) {
    const int b = (bits_packed >> (8 * t)) & 0xff;
    if (b != 2 && b != 4 && b != 8) return ECHOKV_EINVAL;
  }
  // Only the last floor(window / k_group) * k_group keys are scored.
  if (head_size < 1 || head_size > ek::kCanaryMaxD || window < k_group) return ECHOKV_ESHAPE;
  const int rows = (num_q_heads / num_kv_heads) * nq;  // query rows one workgroup scores
  if (ek::canary_lds_bytes(head_size, nbits, rows) > ek::kLdsBytes) return ECHOKV_ESHAPE;
  if (num_layers == 0) return ECHOKV_OK;
  if (!query || !kref || !partial || !out) return ECHOKV_EINVAL;
  ek::CanaryArgs a{query, q_dtype, q_sl, q_s0, q_s1, kref, k_sl, k_s0, k_s1, nq, num_q_heads, num_kv_heads,
                   head_size, window, nbits, bits_packed, k_group, softmax_scale, partial, out};
  return launched(ek::launch_canary(a, num_layers, (hipStream_t)stream));
}

}  // extern "C"
