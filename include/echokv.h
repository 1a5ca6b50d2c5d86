/*
 * echokv.h -- C ABI of the MI355X (gfx950) EchoKV quantized KV-cache hot path.
 *
 * Every entry point launches HIP kernels asynchronously on the given stream and
 * returns 0 on success or an ECHOKV_E* code (no launch happened) on a bad
 * argument. The library never allocates, frees, synchronizes or reads device
 * memory from the host; every buffer is caller-owned, so calls can be captured
 * in a HIP graph. Pointers are device pointers unless noted; strides are in
 * elements. Functions are reentrant: the only process state is a per-device bit
 * recording that a kernel's dynamic-LDS limit was raised (set atomically, by an
 * idempotent call).
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the zimo0110/echokv tree).
 */
#ifndef ECHOKV_H
#define ECHOKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* echokv_stream_t; /* a hipStream_t */

enum { ECHOKV_F32 = 0, ECHOKV_F16 = 1, ECHOKV_BF16 = 2 };

enum {
  ECHOKV_OK = 0,
  ECHOKV_EINVAL = 1,     /* bad pointer / count / stride */
  ECHOKV_ESHAPE = 2,     /* layout or head shape this build does not support */
  ECHOKV_EDTYPE = 3,     /* unsupported dtype code */
  ECHOKV_ELAUNCH = 4,    /* the HIP launch itself failed */
  ECHOKV_ETOOBIG = 5,    /* the request exceeds the library's static scratch buffer */
};

/* echokv_decode flags. */
enum { ECHOKV_DECODE_BATCH_INVARIANT = 1 };

/* One layer's page layout (echokv_vllm/tiered_cache.py:76-147, TieredLayout):
 * header [0, block_size); V scale/min fp16 [block_size, H, D/v_group];
 * K scale/min fp16 [block_size/k_group, H, D]; then chunks_per_page chunks of
 * chunk_bytes = block_size*H*D/2 bytes. Token rows are [K codes | V codes]. */
typedef struct echokv_layout {
  int32_t num_kv_heads, head_size, block_size, k_group, v_group, chunks_per_page;
  int64_t num_blocks;   /* pages in this layer's view */
  int64_t page_stride;  /* bytes between consecutive pages (16-byte multiple) */
  int64_t o_v_scale, o_v_min, o_k_scale, o_k_min, o_data, chunk_bytes;
} echokv_layout;

/* Full-precision K of each block's open group: [rows, k_group, H, D]
 * (echokv_vllm/tiered_cache.py:207-211, TieredKVCache.res_k). */
typedef struct echokv_residual {
  void* ptr;
  int32_t dtype; /* ECHOKV_F32 / F16 / BF16 */
  int32_t rows;  /* residual slots + 1 */
  int64_t s0, s1, s2;
} echokv_residual;

const char* echokv_error_string(int code);

/* Quantize-on-write of one step's token rows: V per token (groups of v_group),
 * K to the residual / under sealed stats / to the K_ref ring.
 * tok: [4, tok_s0] int64 = (slot, residual slot, sealed, kref row) per row; key and
 * value hold n_rows rows, each read whatever its slot (-1 rows included).
 * Replaces echokv_vllm/kernels/write.py:29-36 (write_tokens) and its kernel
 * write.py:172-229 (_write_tokens_kernel). kref may be NULL. */
int echokv_write_tokens(const echokv_layout* L, uint8_t* pages,
                        const void* key, int64_t k_s0, int64_t k_s1,
                        const void* value, int64_t v_s0, int64_t v_s1, int32_t kv_dtype,
                        const int64_t* tok, int64_t tok_s0, int64_t n_rows,
                        const echokv_residual* res, float* kref, int64_t kref_s0, int64_t kref_s1,
                        echokv_stream_t stream);

/* Per-channel quantization of each completed K group.
 * fin: [>= grid_rows, 3 + k_group] int64 = (block, group, residual slot, token row per
 * position or -1 = residual); rows >= *fin_count are skipped (graph full grid).
 * Replaces echokv_vllm/kernels/write.py:39-50 (finalize_k), kernel write.py:232-287. */
int echokv_finalize_k(const echokv_layout* L, uint8_t* pages,
                      const void* key, int64_t k_s0, int64_t k_s1, int32_t kv_dtype,
                      const int64_t* fin, const int64_t* fin_count, int64_t grid_rows,
                      const echokv_residual* res, echokv_stream_t stream);

/* One step's writes in one launch: echokv_finalize_k's fin rows (workgroups
 * [0, fin_grid); fin holds at least fin_grid rows, all of them read, and rows
 * >= *fin_count do nothing) and echokv_write_tokens' token rows
 * (n_rows of them), with the same arguments and results as the finalize-then-write
 * pair. A token whose residual slot is released by a fin row of the same step
 * has its residual K stored by that fin row's workgroup after it has read the
 * slot, so the two launches' order is kept without a second launch.
 * Requires k_group <= 256. Replaces the pair as echokv_vllm/tiered_cache.py:415-432
 * (apply) issues it: finalize_k (write.py:39-50), then write_tokens (write.py:29-36). */
int echokv_write_step(const echokv_layout* L, uint8_t* pages,
                      const void* key, int64_t k_s0, int64_t k_s1,
                      const void* value, int64_t v_s0, int64_t v_s1, int32_t kv_dtype,
                      const int64_t* tok, int64_t tok_s0, int64_t n_rows,
                      const int64_t* fin, const int64_t* fin_count, int64_t fin_grid,
                      const echokv_residual* res, float* kref, int64_t kref_s0, int64_t kref_s1,
                      echokv_stream_t stream);

/* Seal evicted residual groups: ev [n, 6] int64 = (slot, block, group, fill, bits, mask).
 * Replaces the device ops of echokv_vllm/tiered_cache.py:379-394 (_seal). */
int echokv_seal_groups(const echokv_layout* L, uint8_t* pages, const int64_t* ev, int64_t n,
                       const echokv_residual* res, echokv_stream_t stream);

/* The page headers of a step's opened blocks in every layer of a cache group, one
 * launch: layer l's header (16 bytes: tag, then the pool chunk ids) of block ids[i]
 * is headers[(l * n + i) * 16 ..], written at page_bases[l] + ids[i] * page_stride
 * (page_bases: device array of n_layers page-base addresses, 4-byte aligned; ids
 * must name blocks of every layer). Replaces the per-layer header assignment of
 * echokv_vllm/tiered_cache.py:258-307 (open_blocks / write_headers) for a whole step. */
int echokv_write_headers(const uint64_t* page_bases, int32_t n_layers, int64_t page_stride, const int64_t* ids,
                         int64_t n, const uint8_t* headers, echokv_stream_t stream);

/* Dequantized K and V (float32 [n, H, D]) of tokens (blk[i], off[i]); never-opened
 * blocks read as zeros, a block's open K group reads the residual.
 * Replaces echokv_vllm/tiered_cache.py:451-478 (gather). */
int echokv_gather(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                  const int64_t* res_group, const echokv_residual* res,
                  const int64_t* blk, const int64_t* off, int64_t n,
                  float* k_out, float* v_out, echokv_stream_t stream);

/* Requantize whole blocks from float32 K, V [n*block_size, H, D] at `bits`, setting
 * the tag byte (K per channel over K groups, V per token).
 * Replaces the device ops of echokv_vllm/tiered_cache.py:322-340 (_demote_lru). */
int echokv_store_blocks(const echokv_layout* L, uint8_t* pages, const int64_t* blocks, int64_t n,
                        const float* k, const float* v, int32_t bits, echokv_stream_t stream);

/* Paged decode attention: sequence i attends with query row q_rows[i] (NULL = i)
 * over block-table row bt_rows[i] (NULL = i) for seq_lens[i] tokens and writes
 * out[q_rows[i]]; seq_lens[i] == 0 leaves the row untouched. acc: [rows, Hq, D]
 * f32 and ml: [rows, Hq, 2] f32 workspaces, rows = echokv_decode_workspace_rows(...)
 * of the same arguments (at most num_seqs * num_splits).
 * Default schedule: the batch's blocks are cut into equal ranges, one per workgroup
 * the chip holds (at most num_seqs * num_splits / 2); a sequence inside one range is
 * written directly, the others merged from partials. With flags &
 * ECHOKV_DECODE_BATCH_INVARIANT: split-KV with splits of
 * max(blocks_per_split, ceil(blocks / num_splits)) blocks of the sequence's own
 * length, so a sequence's result does not depend on the rest of the batch. tier
 * (2, 4 or 8) selects the kernel specialised for the layer's tier; blocks stored at
 * another tier, and each block's open K group, are still read correctly on a slower
 * path. tier_mask (device int32, or NULL) names the tiers the layer holds blocks at,
 * as a bit set of tier values (2 | 4 | 8; 0 reads as `tier` alone), read when the
 * kernels run (a captured graph follows it): the kernel of each of those tiers runs
 * that tier's blocks on its own fast path, one after another into the same
 * partial rows, and one merge follows. It needs ECHOKV_DECODE_BATCH_INVARIANT
 * (the split schedule), and a sequence's result still depends on its own blocks
 * only. Layouts: head_size 64 or 128 with v_group >= head_size / 16, or head_size
 * 256 with v_group 8 to 128 (each KV head as two 128-channel halves), k_group >= 16,
 * power-of-two block_size and k_group and <= 4 chunks per page run on the MFMA
 * kernels; any other layout (head_size up to 256) on an fp32 kernel with the split
 * schedule (flags and tier then select nothing).
 * Replaces echokv_vllm/kernels/decode.py:44-92 (decode_attention) with its kernels
 * decode.py:135-224 (_decode_kernel) and decode.py:227-262 (_merge_kernel). */
int echokv_decode(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                  const int64_t* res_group, const echokv_residual* res,
                  const void* query, int64_t q_s0, int64_t q_s1, int32_t q_dtype, int32_t num_q_heads,
                  const int64_t* q_rows, const int32_t* block_table, int64_t bt_s0,
                  const int64_t* bt_rows, const int64_t* seq_lens, int64_t num_seqs,
                  float softmax_scale, int32_t num_splits, int32_t blocks_per_split, int32_t tier,
                  const int32_t* tier_mask, int32_t flags, float* acc, float* ml, void* out, int64_t o_s0,
                  int64_t o_s1, int32_t out_dtype, echokv_stream_t stream);

/* Rows of the acc / ml workspaces that echokv_decode uses with these arguments,
 * for any tier: num_seqs * num_splits for the split schedule, two per range of the
 * balanced one (ranges follow the kernels' occupancy on the current device). -1
 * for arguments echokv_decode would refuse. No counterpart in the reference: its
 * launcher allocates [S, Hq, splits, D] per call (echokv_vllm/kernels/decode.py:306-307). */
int64_t echokv_decode_workspace_rows(const echokv_layout* L, int32_t num_q_heads, int32_t q_dtype,
                                     int64_t num_seqs, int32_t num_splits, int32_t flags);

/* echokv_decode without workspace arguments, for callers that cannot allocate
 * (code under HIP-graph capture, serving loops that forbid allocation): acc and
 * ml live in a static device array of the library (64 MiB per GPU, held until the
 * process ends), so num_seqs * num_q_heads * num_splits * (head_size + 2) * 4
 * must be at most 64 MiB, else ECHOKV_ETOOBIG and nothing is launched. The call
 * allocates nothing. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams, or host threads) race and must be
 * ordered by the caller. No counterpart in the reference. */
int echokv_decode_static(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                         const int64_t* res_group, const echokv_residual* res,
                         const void* query, int64_t q_s0, int64_t q_s1, int32_t q_dtype, int32_t num_q_heads,
                         const int64_t* q_rows, const int32_t* block_table, int64_t bt_s0,
                         const int64_t* bt_rows, const int64_t* seq_lens, int64_t num_seqs,
                         float softmax_scale, int32_t num_splits, int32_t blocks_per_split, int32_t tier,
                         const int32_t* tier_mask, int32_t flags, void* out, int64_t o_s0, int64_t o_s1,
                         int32_t out_dtype, echokv_stream_t stream);

/* Chunked-prefill attention over the tiered pages (MFMA tiles), bottom-right causal:
 * tiles [n_tiles, 5] int32 = (first query row, tokens, first query position, ctx,
 * block-table row); each tile holds <= tile_m query tokens: tile_m = 128 / GQA on the
 * MFMA kernel (head size 64 or 128, GQA <= 128; 64 / GQA at head size 256, GQA <= 64),
 * else 16 / GQA (1 from GQA 16 on) on an fp32 kernel for head sizes up to 256 (no
 * own_group there). own_group = 1 leaves
 * each query's own K group out (a query at p sees keys < p & ~(k_group - 1); k_group
 * a power of two); lse (nullable, float [query rows, num_q_heads]) receives each
 * row's log2-domain log-sum-exp of the scaled scores (-inf: no visible key).
 * Replaces echokv_vllm/kernels/prefill.py:170-207 (prefill_attention: the fused kernel
 * prefill.py:242-327 and the dense dequant + flash-attention path prefill.py:133-167). */
int echokv_prefill(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                   const int64_t* res_group, const echokv_residual* res,
                   const void* query, int64_t q_s0, int64_t q_s1, int32_t q_dtype, int32_t num_q_heads,
                   void* out, int64_t o_s0, int64_t o_s1, int32_t out_dtype,
                   const int32_t* tiles, int64_t n_tiles, int32_t tile_m,
                   const int32_t* block_table, int64_t bt_s0, float softmax_scale,
                   int32_t own_group, float* lse, echokv_stream_t stream);

/* Long-chunk prefill in two passes (the dense path for chunks longer than the fused
 * kernel's): each 64-key tile of every context is dequantized once into `workspace`
 * (packs [n_packs, 3] int32 = (block-table row, first key, ctx); tile i of head h at
 * byte (i * H + h) * 64 * D * 6: K rows as fp16 hi + lo, V transposed fp16), then
 * flash attention on MFMA reads it: qtiles [n_qtiles, 5] int32 = (first query row,
 * tokens <= tile_m = 256 / GQA, first query position, ctx, first workspace tile of
 * the request's context), bottom-right causal. Workspace reads stay below n_packs tiles.
 * own_group / lse as for echokv_prefill.
 * Replaces echokv_vllm/kernels/prefill.py:133-167 (prefill_attention_dense:
 * dequant_dense prefill.py:90-115 + flash-attention varlen).
 * echokv_prefill_dense_workspace: the workspace bytes for n_packs tiles, or minus an
 * error code. */
int64_t echokv_prefill_dense_workspace(const echokv_layout* L, int64_t n_packs);
int echokv_prefill_dense(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                         const int64_t* res_group, const echokv_residual* res,
                         const void* query, int64_t q_s0, int64_t q_s1, int32_t q_dtype, int32_t num_q_heads,
                         void* out, int64_t o_s0, int64_t o_s1, int32_t out_dtype,
                         const int32_t* packs, int64_t n_packs, const int32_t* qtiles, int64_t n_qtiles,
                         int32_t tile_m, const int32_t* block_table, int64_t bt_s0,
                         void* workspace, int64_t workspace_bytes, float softmax_scale,
                         int32_t own_group, float* lse, echokv_stream_t stream);

/* Own-group-exact prefill, second part: each query attends to its own K group with
 * full-precision keys -- this step's key rows (key, aligned with the query rows)
 * at positions >= the chunk's first position, the cache before it -- and cached V,
 * as decode saw the group while it was open; the result merges by log-sum-exp with
 * part (fp32 [query rows, num_q_heads, D], strides p_s0 / p_s1) and lse, the output
 * of echokv_prefill / echokv_prefill_dense with own_group = 1, into out.
 * rows [n_rows, 4] int32 = (query row, position, chunk's first position, block-table
 * row). k_group <= 64 (a power of two), head_size <= 128, GQA <= 16.
 * No counterpart in the reference: its docs/ECHOKV_VLLM_PLUGIN.md:261-266 names this
 * fix for preempted / re-chunked requests (prefill sees its own group quantized where
 * decode saw it exact) and leaves it open. */
int echokv_prefill_own_group(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                             const int64_t* res_group, const echokv_residual* res,
                             const void* query, int64_t q_s0, int64_t q_s1, int32_t q_dtype, int32_t num_q_heads,
                             const void* key, int64_t k_s0, int64_t k_s1, int32_t k_dtype,
                             const int32_t* rows, int64_t n_rows, const int32_t* block_table, int64_t bt_s0,
                             const float* part, int64_t p_s0, int64_t p_s1, const float* lse,
                             void* out, int64_t o_s0, int64_t o_s1, int32_t out_dtype,
                             float softmax_scale, echokv_stream_t stream);

/* Dense dequantization of prefill contexts: work [n, 4] int32 = (block-table row,
 * block index, dense row of the block's first token, ctx) -> K, V [*, H, D].
 * Replaces echokv_vllm/kernels/prefill.py:90-115 (dequant_dense), kernel 330-369. */
int echokv_dequant_dense(const echokv_layout* L, const uint8_t* pages, const int64_t* block_res,
                         const int64_t* res_group, const echokv_residual* res,
                         const int32_t* work, int64_t n_work, const int32_t* block_table, int64_t bt_s0,
                         void* k_out, void* v_out, int64_t o_s0, int64_t o_s1, int32_t out_dtype,
                         echokv_stream_t stream);

/* Canary: for each layer and tier bits[j], the mean over query rows and heads of
 * KL(softmax(q K~ᵀ s) || softmax(q K_refᵀ s)), K~ = per-channel storage round trip
 * of the last floor(window/k_group)*k_group keys; clamped >= 0. Any window length.
 * query [L, nq, Hq, D] (strides q_sl, q_s0, q_s1), kref f32 [L, window, H, D]
 * oldest first (strides k_sl, k_s0, k_s1) -> out f32 [L, nbits]; tier j is byte j of
 * bits_packed (each 2, 4 or 8). partial: f32 workspace [L, H, nbits] (the KL sums of
 * each layer's KV heads, added in head order). D <= 256.
 * Replaces echokv_vllm/canary.py:59-89 (canary_kl). */
int echokv_canary_kl(const void* query, int32_t q_dtype, int64_t q_sl, int64_t q_s0, int64_t q_s1,
                     const float* kref, int64_t k_sl, int64_t k_s0, int64_t k_s1,
                     int32_t num_layers, int32_t nq, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_size, int32_t window, int32_t nbits, int32_t bits_packed, int32_t k_group,
                     float softmax_scale, float* partial, float* out, echokv_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* ECHOKV_H */
