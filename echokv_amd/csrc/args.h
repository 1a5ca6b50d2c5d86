// Kernel argument structs (passed by value) and launchers of libechokv.
#pragma once

#include <atomic>

#include "common.h"

namespace ek {

constexpr int kThreads = 256;        // store / dequant kernels
constexpr int kCanaryMaxTiers = 3;
constexpr int kCanaryMaxD = 256;
constexpr size_t kLdsBytes = 160 * 1024;  // LDS per CU on gfx950
constexpr int kPrefillRows = 128;    // prefill: query rows (tokens x GQA heads) per workgroup

// Query rows of a prefill workgroup (head size 256: half, one 16-row block per
// wave) and query tokens per tile for a GQA group size.
inline int prefill_rows(int head_size) { return head_size == 256 ? kPrefillRows / 2 : kPrefillRows; }
inline int prefill_tile_tokens(int gqa, int head_size) { return prefill_rows(head_size) / gqa; }

// Long-chunk (two-pass) prefill: keys per workspace tile, waves (32 query rows
// each) per attention workgroup, and the workspace bytes of one tile and head.
constexpr int kDenseKeys = 64;
constexpr int kDenseWaves = 8;
inline int dense_tile_tokens(int gqa) { return 32 * kDenseWaves / gqa; }
// A tile holds K as fp16 hi + fp8 lo (3 bytes per channel) and V^T as fp16, padded to
// whole rounds of the attention kernel's 1 KiB-per-wave DMAs.
inline long dense_tile_bytes(int D) {
  const long raw = (long)kDenseKeys * D * 5, round = 1024L * kDenseWaves;
  return (raw + round - 1) / round * round;
}

struct WriteTokArgs {
  Lay L;
  uint8_t* pages;
  const void* key;
  long k_s0, k_s1;
  const void* value;
  long v_s0, v_s1;
  int kv_dtype;
  const int64_t* tok;
  long tok_s0;
  Res res;
  float* kref;
  long kref_s0, kref_s1;
};

struct FinArgs {
  Lay L;
  uint8_t* pages;
  const void* key;
  long k_s0, k_s1;
  int kv_dtype;
  const int64_t* fin;
  const int64_t* fin_count;
  Res res;
};

// A fused step: token rows plus fin rows (fin: [>= fin_grid, 3 + KG], every row
// below fin_grid is read; rows at or past *fin_count do nothing).
constexpr int kMaxDeferred = 256;  // k_group bound of the fused step (a slot's group has < k_group rows in a step)
struct StepArgs {
  WriteTokArgs w;
  const int64_t* fin;
  const int64_t* fin_count;
  long fin_grid;
  long n_rows;
  int staged;  // dtype of key and residual when fin rows stage their group in LDS, else -1
  // > 0: each fin row is split over fin_parts workgroups of 64 (head, quad) items,
  // its K group over 4 lanes per item (staged dtype, k_group 8 to 64); 0: one
  // workgroup per fin row.
  int fin_parts;
};

// Dynamic LDS of a staged fused step, and the largest the launch takes without
// raising the kernel's limit.
inline size_t step_staged_lds(int k_group, int dtype) {
  return (size_t)k_group * kThreads * (dtype == ECHOKV_F32 ? 16 : 8);
}
constexpr size_t kStepStagedMaxLds = 64 * 1024;

// The keys a prefill query at position p sees are those < og_limit(p): p + 1
// (bottom-right causal), or with own_group on (og_mask = ~(k_group - 1)) the keys
// before its own K group -- unless p closes the group: decode read that group
// back quantized, so the whole prefix stays.
__device__ __forceinline__ int og_limit(int p, int og_mask) {
  return og_mask && ((p + 1) & ~og_mask) ? (p & og_mask) : p + 1;
}

// Own-group attention of prefill chunks (own_group_kernel): rows [n, 4] =
// (query row, position, chunk's first position c0, block-table row).
constexpr int kOgMaxKeys = 64, kOgMaxD = 128, kOgMaxGqa = 16;
struct OwnGroupArgs {
  Lay L;
  const uint8_t* pages;
  const int64_t* block_res;
  const int64_t* res_group;
  Res res;
  const void* q;
  long q_s0, q_s1;
  int q_dtype, hq, gqa;
  const void* key;
  long k_s0, k_s1;
  int k_dtype;
  const int32_t* rows;
  const int32_t* bt;
  long bt_s0;
  const float* part;  // [q rows][hq][D] fp32: attention over the keys before each query's group
  long p_s0, p_s1;
  const float* lse;   // [q rows][hq]: its log2-domain log-sum-exp (-inf: no such key)
  void* out;
  long o_s0, o_s1;
  int out_dtype;
  float scale_log2;
};

struct SealArgs {
  Lay L;
  uint8_t* pages;
  const int64_t* ev;
  Res res;
};

struct StoreBlkArgs {
  Lay L;
  uint8_t* pages;
  const int64_t* blocks;
  const float* k;
  const float* v;
  int bits;
};

struct GatherArgs {
  Lay L;
  const uint8_t* pages;
  const int64_t* block_res;
  const int64_t* res_group;
  Res res;
  const int64_t* blk;
  const int64_t* off;
  float* k_out;
  float* v_out;
};

struct DenseArgs {
  Lay L;
  const uint8_t* pages;
  const int64_t* block_res;
  const int64_t* res_group;
  Res res;
  const int32_t* work;
  const int32_t* bt;
  long bt_s0;
  void* k_out;
  void* v_out;
  long o_s0, o_s1;
  int out_dtype;
};

struct DecodeArgs {
  Lay L;
  const uint8_t* pages;
  const int64_t* block_res;
  const int64_t* res_group;
  Res res;
  const void* q;
  long q_s0, q_s1;
  int q_dtype, hq, gqa;
  int g0, gs;  // this pass's query heads of each KV head: [g0, g0 + gs), gs <= 16
  // 1: the V scale rides on the P operand (gs * (D / VG) <= 16, D / VG <= 4): the
  // MFMA columns are (query head, V group) pairs; 0: V is dequantized per element.
  int ps;
  const int64_t* q_rows;
  const int32_t* bt;
  long bt_s0;
  const int64_t* bt_rows;
  const int64_t* lens;
  float scale_log2;  // softmax scale * log2(e)
  int num_splits, bps;
  long num_seqs;
  int tier;    // the layer's tier: selects the kernel specialised for it (2, 4 or 8)
  // Tier passes (split schedule): null, or the layer's tiers with live blocks as a
  // bit set of tier values (2 | 4 | 8; 0: `tier0` alone). Each kernel of the tiers
  // 2, 4, 8 then runs its tier's blocks only; the lowest present tier also takes
  // blocks of tiers outside the set and starts each span afresh, the others
  // continue the span's partial result that the pass before them left.
  const int32_t* tier_mask;
  int tier0;
  // 1: head size 256 run as half-heads. L is then the layer seen as 2 * H heads of
  // D / 2 channels (the same bytes: a token row holds each head's codes, and each
  // statistic array each head's channels or V groups, side by side), and half-heads
  // 2k and 2k + 1 are the channel halves of KV head k: they share its query heads,
  // add their partial scores before the softmax, and write the two halves of its
  // rows (acc rows then hold 2 * L.D floats).
  int pair;
  // log2 of block size, K group and V group (powers of two), and a reciprocal for
  // chunk id / chunks_per_page: floor(id / KC) = umulhi(id, kc_mul) (kc_mul 0: KC = 1).
  int bs_shift, kg_shift, vg_shift;
  uint32_t kc_mul;
  float* acc;  // [S, Hq, splits, D]
  float* ml;   // [S, Hq, splits, 2] = (running max in log2 units, sum)
  // Balanced schedule (ranges > 0): `ranges` equal block ranges; partial slot p of
  // query head qh is row p * Hq + qh of acc / ml (2 * ranges slots); sequences
  // inside one range are written to `out` directly. 0: the split schedule.
  long ranges;
  void* out;
  long o_s0, o_s1;
  int out_dtype;
};

struct MergeArgs {
  const float* acc;
  const float* ml;
  const int64_t* lens;
  const int64_t* q_rows;
  void* out;
  long o_s0, o_s1;
  int out_dtype, hq, D, BS, num_splits, bps;
  long rows;  // num_seqs * hq
  int gqa, g0, gs;  // rows of query heads g0 .. g0 + gs - 1 of each KV head only
};

struct CanaryArgs {
  const void* q;
  int q_dtype;
  long q_sl, q_s0, q_s1;
  const float* kref;
  long k_sl, k_s0, k_s1;
  int nq, hq, h, d, window, nbits, bits_packed, kg;
  float scale;
  float* partial;  // [layers, H, nbits]: KL sums of each (layer, KV head)
  float* out;
};

struct PrefillArgs {
  Lay L;
  const uint8_t* pages;
  const int64_t* block_res;
  const int64_t* res_group;
  Res res;
  const void* q;
  long q_s0, q_s1;
  int q_dtype, hq, gqa;
  void* out;
  long o_s0, o_s1;
  int out_dtype;
  const int32_t* tiles;  // [n, 5]: first query row, tokens, first query position, ctx, block-table row
  const int32_t* bt;
  long bt_s0;
  float scale_log2;
  int og_mask;  // nonzero: a query at position p sees keys < (p & og_mask) (its own K group left out)
  float* lse;   // nullable: [rows, hq] log2-domain log-sum-exp of each query row's scores
  int g0, gs;   // fp32 kernel (prefill_any): this pass's query heads of each KV head, gs <= 16
};

struct PackArgs {
  Lay L;
  const uint8_t* pages;
  const int64_t* block_res;
  const int64_t* res_group;
  Res res;
  const int32_t* packs;  // [n, 3]: block-table row, first key, ctx
  const int32_t* bt;
  long bt_s0;
  uint8_t* ws;  // [n][H][dense_tile_bytes(D)]
};

struct FlashArgs {
  const uint8_t* ws;
  const void* q;
  long q_s0, q_s1;
  int q_dtype;
  void* out;
  long o_s0, o_s1;
  int out_dtype;
  const int32_t* qtiles;  // [n, 5]: first query row, tokens, first query position, ctx, first workspace tile
  int n_qtiles, H, gqa, D;
  long n_packs;  // workspace tiles present: reads stay below this
  float scale_log2;
  int og_mask;  // as PrefillArgs::og_mask
  float* lse;   // as PrefillArgs::lse
  int hq;
};

// Raise `kernel`'s dynamic-LDS limit to `bytes` on the current device, once per
// device. The flag only skips a repeated call: hipFuncSetAttribute is idempotent,
// so two threads that race on a fresh device both make it and both succeed.
template <int kMaxDevices = 64>
inline hipError_t ensure_lds_limit(const void* kernel, int bytes, std::atomic<uint64_t>* done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return hipErrorInvalidDevice;
  const uint64_t bit = 1ull << (dev % kMaxDevices);
  if (done->load(std::memory_order_acquire) & bit) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done->fetch_or(bit, std::memory_order_release);
  return e;
}

// Static scratch of echokv_decode_static (decode.hip): its size, and its address on
// the current device (resolved once per device).
constexpr size_t kDecodeScratchBytes = 64u << 20;
hipError_t decode_scratch(void** ptr);

hipError_t launch_write_tokens(const WriteTokArgs& a, long n_rows, hipStream_t s);
hipError_t launch_finalize_k(const FinArgs& a, long rows, hipStream_t s);
hipError_t launch_write_step(const StepArgs& a, hipStream_t s);
hipError_t launch_own_group(const OwnGroupArgs& a, long n, hipStream_t s);
hipError_t launch_seal(const SealArgs& a, long n, hipStream_t s);
hipError_t launch_store_blocks(const StoreBlkArgs& a, long n, hipStream_t s);
hipError_t launch_gather(const GatherArgs& a, long n, hipStream_t s);
hipError_t launch_write_headers(const uint64_t* page_bases, long page_stride, const int64_t* ids,
                                const uint32_t* hdr, int n_layers, long n, hipStream_t s);
hipError_t launch_dequant_dense(const DenseArgs& a, long n, hipStream_t s);
hipError_t launch_decode(const DecodeArgs& a, long num_seqs, hipStream_t s);
// Ranges of the balanced schedule for a batch on the current device: one per
// workgroup slot the chip holds for the layer's tier, at most num_seqs * num_splits / 2.
hipError_t decode_ranges(const DecodeArgs& a, long& ranges);
hipError_t launch_merge_balanced(const DecodeArgs& a, hipStream_t s);
hipError_t launch_merge(const MergeArgs& a, long num_seqs, hipStream_t s);
// Decode for the layouts the MFMA kernels do not take (decode_any.hip): split
// schedule only, head size a multiple of 4 up to kMaxAnyD.
constexpr int kMaxAnyD = 256;
hipError_t launch_decode_any(const DecodeArgs& a, hipStream_t s);
hipError_t launch_merge_any(const MergeArgs& a, hipStream_t s);
// Prefill for those layouts: tiles of any_tile_tokens(gqa) query tokens, one
// workgroup per (tile, KV head), each query's causal context streamed once per tile.
inline int any_tile_tokens(int gqa) { return gqa >= 16 ? 1 : 16 / gqa; }
hipError_t launch_prefill_any(const PrefillArgs& a, long n_tiles, hipStream_t s);
hipError_t launch_canary(const CanaryArgs& a, int num_layers, hipStream_t s);
size_t canary_lds_bytes(int d, int nbits, int rows);  // one canary workgroup's LDS
hipError_t launch_prefill(const PrefillArgs& a, long n_tiles, hipStream_t s);
hipError_t launch_prefill_pack(const PackArgs& a, long n_packs, hipStream_t s);
hipError_t launch_prefill_flash(const FlashArgs& a, hipStream_t s);

}  // namespace ek
