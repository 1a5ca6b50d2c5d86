/*
 * echokv_host.h -- C ABI of the native host side of the tiered KV store: the
 * per-step write planner (shared by the layers of one KV-cache group) and each
 * layer's chunk pool. CPU only (libechokv_host.so, built with g++); called from
 * Python with ctypes. Objects are not thread-safe: one caller thread per object.
 *
 * Each entry point names the reference interface it replaces (paths relative to
 * the zimo0110/echokv tree).
 */
#ifndef ECHOKV_HOST_H
#define ECHOKV_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { EKH_OK = 0, EKH_EINVAL = 1, EKH_ESLOTS = 2 /* more open K groups than residual slots */ };

typedef struct ekh_planner ekh_planner;
typedef struct ekh_pool ekh_pool;

/* The result of one ekh_plan call; the pointers stay valid until the next call.
 * stage: one int64 image, copied to the device as is:
 *   [n_fin | tok: slot, residual slot, sealed, K_ref row (4 x n_rows) |
 *    fin (n_fin x (3 + k_group)) | residual map: blocks, values (n_res_map each) |
 *    residual groups: slots, groups (n_grp_map each)]
 * fin rows: (block, group, residual slot or -1, token row per position or -1).
 * evict [n_evict, 4] = (slot, block, group, fill); open [n_open] ascending;
 * touched [n_touched, 3] = (block, highest offset written + 1, tokens). */
typedef struct ekh_plan_view {
  int64_t step, n_rows, n_fin, n_evict, n_open, n_touched, n_res_map, n_grp_map, stage_len;
  const int64_t* stage;
  const int64_t* evict;
  const int64_t* open;
  const int64_t* touched;
} ekh_plan_view;

/* Planner + per-block host bookkeeping (fill, last step written, tokens written);
 * num_blocks <= 0: the per-block arrays grow with the slots seen (no pool may then
 * use the planner, and ekh_block_array pointers change as they grow).
 * Replaces echokv_vllm/write_plan.py:77-96 (WritePlanner.__init__, _release) and 243-256
 * (SharedState's host arrays). NULL on bad sizes. */
ekh_planner* ekh_planner_new(int64_t num_blocks, int32_t block_size, int32_t k_group, int32_t residual_slots,
                             int32_t kref_window);
void ekh_planner_free(ekh_planner* p);

/* Plan one step's writes from its slot mapping (-1 = no write).
 * Replaces echokv_vllm/write_plan.py:98-240 (WritePlanner.plan) and the host
 * half of write_plan.py:285-315 (stage_plan: the image to upload). */
int ekh_plan(ekh_planner* p, const int64_t* slot_mapping, int64_t n_rows, ekh_plan_view* out);

/* Record a planned step's touched blocks [n, 3] (block, fill, count) in the
 * per-block bookkeeping. Replaces echokv_vllm/write_plan.py:258-264 (SharedState.commit). */
int ekh_commit(ekh_planner* p, int64_t step, const int64_t* touched, int64_t n_touched);

enum { EKH_STEP = 0, EKH_RES_FREE = 1, EKH_RES_SLOTS = 2, EKH_KREF_POS = 3, EKH_KREF_FILL = 4, EKH_KREF_WINDOW = 5,
       EKH_NUM_BLOCKS = 6 };
/* Planner counters (write_plan.py:81-90 attributes); -1 for an unknown field. */
int64_t ekh_planner_state(const ekh_planner* p, int32_t what);
/* The residual free list, bottom to top (the top is handed out next); returns its length. */
int64_t ekh_residual_free_list(const ekh_planner* p, int64_t* out, int64_t cap);
/* Bit g set: K group g of `block` was sealed by an eviction (write_plan.py:85). */
int32_t ekh_sealed_mask(const ekh_planner* p, int64_t block);

enum { EKH_FILL = 0, EKH_LAST = 1, EKH_CUM = 2 };
/* The per-block arrays [num_blocks] int64 (SharedState.fill_h / last_h / cum_h). */
int64_t* ekh_block_array(ekh_planner* p, int32_t which);

/* One layer's chunk pool over the planner's bookkeeping (a planner with a block count).
 * Replaces echokv_vllm/tiered_cache.py:196-202, 224-226 (the pool and counters of TieredKVCache). */
ekh_pool* ekh_pool_new(ekh_planner* planner, int32_t chunks_per_page);
void ekh_pool_free(ekh_pool* q);

/* (Re)open `blocks` at target_bits or the best tier the pool allows; writes
 * headers [n, 16] and, when the pool ran short, the least recently written full
 * blocks it chose to demote (victims, at most num_blocks; the caller requantizes
 * them to INT2 on the device before writing the headers).
 * Replaces echokv_vllm/tiered_cache.py:258-303 (open_blocks) and the host half
 * of 309-346 (_demote_lru). */
int ekh_pool_open(ekh_pool* q, const int64_t* blocks, int64_t n, int32_t target_bits, const int64_t* protect,
                  int64_t n_protect, uint8_t* headers, int64_t* victims, int64_t* n_victims);

/* The device row (slot, block, group, fill, bits, mask) sealing eviction
 * ev = (slot, block, group, fill). Replaces the host half of
 * echokv_vllm/tiered_cache.py:379-394 (_seal). */
int64_t ekh_pool_seal_row(ekh_pool* q, const int64_t* ev, int64_t* row);

/* out[23]: tokens written per tier [9], blocks opened per tier [9], downgraded,
 * demoted, sealed groups, free chunks, pool size.
 * Replaces echokv_vllm/tiered_cache.py:230-252 (_settle, tokens_written, pool_free). */
void ekh_pool_counters(const ekh_pool* q, int64_t* out);
/* Replaces echokv_vllm/tiered_cache.py:240-246 (reset_counters). */
void ekh_pool_reset_counters(ekh_pool* q);
/* Each block's host-side tier [num_blocks] int64 (0 = never opened). */
int64_t* ekh_pool_tags(ekh_pool* q);
/* The chunk free list, bottom to top; returns its length. */
int64_t ekh_pool_free_list(const ekh_pool* q, int64_t* out, int64_t cap);
/* Blocks stored at each tier now, out[9] (index 0: never opened). */
void ekh_pool_live(const ekh_pool* q, int64_t* out);

/* ---- per-step driver of a KV-cache group ------------------------------------ */

/* One engine step's batch, as vLLM's CommonAttentionMetadata gives it. */
typedef struct ekh_batch {
  int64_t num_reqs, num_tokens;
  const int32_t* query_start;  /* [num_reqs + 1] */
  const int32_t* seq_lens;     /* [num_reqs], the step's tokens included */
  const int64_t* slot_mapping; /* [num_tokens], -1 = no write */
} ekh_batch;

/* Where each part of a step image sits (int64 words from its start) and how
 * much of it the step uses. The image:
 *   [0] fin rows, [1] token rows;
 *   canary rows [canary_slots] at o_canary;
 *   each layer's tiers with live blocks, as 2 | 4 | 8 (one word per layer) at o_mask;
 *   decode query rows, block-table rows, lengths (rows_dec each) at o_dec;
 *   token rows: slot, residual slot, sealed, K_ref row (rows_tok each) at o_tok;
 *   fin rows [rows_fin, 3 + k_group] at o_fin;
 *   residual map: blocks, values (n_res each) at o_res;
 *   residual groups: slots, groups (n_grp each) at o_grp;
 *   opened block ids [n_open] at o_open;
 *   page headers [layers, n_open, 16 bytes] at o_hdr;
 *   seal rows [layers, n_seal, 6] at o_seal (the rows ekh_pool_seal_row makes).
 * For a step of at most `cap` decode entries, token rows and fin rows
 * (graph_rows = 1) rows_* equal the capacity, so everything up to o_res sits at
 * fixed offsets. */
typedef struct ekh_step_view {
  int64_t step, len, o_canary, o_mask, o_dec, o_tok, o_fin, o_res, o_grp, o_open, o_hdr, o_seal;
  int64_t rows_dec, rows_tok, rows_fin;
  int64_t n_dec, n_tokens, n_fin, n_res, n_grp, n_open, n_seal, n_canary, decode_only, graph_rows;
  double canary_ctx;          /* mean context of the canary's requests */
  int64_t n_prefill;
  const int64_t* prefill;     /* [n_prefill, 4]: query start, query end, context, request */
  int64_t n_victims;
  const int64_t* victims;     /* [n_victims, 2]: layer, block -- requantize to INT2 before the headers */
  const int64_t* image;       /* the caller's buffer, or the stepper's own when it was too small */
} ekh_step_view;

typedef struct ekh_stepper ekh_stepper;

/* A driver over a planner and its layers' pools (all built on that planner);
 * `cap`: the graph capacity in rows, `canary_slots`: query rows a fire stashes. */
ekh_stepper* ekh_stepper_new(ekh_planner* planner, ekh_pool* const* pools, int32_t n_layers, int64_t cap,
                             int32_t canary_slots);
void ekh_stepper_free(ekh_stepper* s);

/* Plan one step for every layer and write its image into `image` (or the
 * stepper's own buffer when image_cap is too small). tiers[layer]: the tier
 * blocks opened now take in that layer; fire: take the canary rows this step.
 * Replaces the host side of echokv_vllm/backend.py:337-496 (the builder's
 * batch layout, _plan and _Staging's image) and write_plan.py:98-240. */
int ekh_stepper_run(ekh_stepper* s, const ekh_batch* batch, const int32_t* tiers, int32_t fire, int64_t* image,
                    int64_t image_cap, ekh_step_view* out);

/* vLLM's slot mapping computed on the host from a host copy of the block table
 * ([table_rows, table_cols] int32, row stride table_stride) and the host
 * sequence lengths: slot = table[row][pos / bs] * bs + pos % bs, where row is
 * the batch row or row_map[batch row]; rows past the scheduled tokens get -1.
 * EKH_EINVAL when the host copies cannot stand in for the device mapping.
 * Replaces echokv_vllm/host_slots.py:170-195 (host_lens_and_slots). */
int ekh_host_slots(const ekh_batch* batch, const int32_t* table, int64_t table_rows, int64_t table_cols,
                   int64_t table_stride, const int64_t* row_map, int64_t row_map_len, int32_t block_size,
                   int64_t* slots);

#ifdef __cplusplus
}
#endif
#endif /* ECHOKV_HOST_H */
