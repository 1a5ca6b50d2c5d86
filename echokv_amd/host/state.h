// Internal state of the native host side (not part of the C ABI): the write
// planner shared by a KV-cache group's layers and each layer's chunk pool.
// plan.cpp implements the planner and pool entry points, step.cpp the
// per-step driver that runs both for every layer and lays out the step image.
#ifndef ECHOKV_HOST_STATE_H
#define ECHOKV_HOST_STATE_H

#include <stdint.h>

#include <algorithm>
#include <vector>

namespace ekh {

constexpr int kExtra[9] = {0, 0, 0, 0, 1, 0, 0, 0, 3};  // pool chunks per tier beyond chunk 0

struct Planner {
  int64_t nb = 0;
  bool growable = false;  // created without a block count: per-block arrays grow on demand
  int bs = 0, kg = 0, gpb = 0, R = 0, W = 0;
  // Residual slots.
  std::vector<int32_t> free_stack;  // back() is handed out next
  std::vector<int64_t> s_block, s_last, s_taken, s_prot;
  std::vector<int32_t> s_group, s_fill;
  std::vector<uint8_t> s_used;
  std::vector<int32_t> block_slot;  // -1: no open group in the residual
  std::vector<uint8_t> sealed;      // bit g: K group g sealed by an eviction
  int64_t step = 0, taken = 0, kref_pos = 0, kref_fill = 0;
  // Per-block bookkeeping read by the pools (tiered_cache.py:243-271).
  std::vector<int64_t> fill_h, last_h, cum_h;

  // The last plan (plan_rows): per token row, the fin rows (whole groups first),
  // the residual map and group updates, evictions (slot, block, group, fill),
  // opened blocks (ascending) and touched blocks (block, fill, count).
  int64_t n_rows = 0, n_fin = 0;
  std::vector<int64_t> tok_res, tok_sealed, tok_kref, fin;
  std::vector<int64_t> evict, opens, touched, res_b, res_v, grp_s, grp_g;
  std::vector<int64_t> stage;  // ekh_plan's image
  std::vector<int64_t> res_stamp, res_at, grp_stamp, grp_at;  // first-appearance position this step
  // Scratch.
  std::vector<int64_t> rows, key, order;

  void grow(int64_t need);
  void res_op(int64_t b, int64_t v);
  void grp_op(int32_t s, int32_t g);
  void release(int32_t s);
  int32_t victim() const;
  int32_t take(int64_t b, int32_t g);
};

struct Pool {
  Planner* p = nullptr;
  int64_t nb = 0;
  int kc = 0, bs = 0;
  std::vector<int64_t> free_chunks;  // back() is handed out next
  int64_t pool_size = 0;
  std::vector<int64_t> tag, table, mark;  // table: [nb, 3]
  int64_t tok_tier[9] = {};
  int64_t opened[9] = {};
  int64_t live[9] = {};  // blocks currently stored at each tier (index 0: never opened)
  int64_t downgraded = 0, demoted = 0, sealed_groups = 0;

  void settle(int64_t b) {
    tok_tier[tag[b]] += p->cum_h[b] - mark[b];
    mark[b] = p->cum_h[b];
  }
  void give_back(int64_t b) {
    for (int j = 0; j < kExtra[tag[b]]; ++j) free_chunks.push_back(table[3 * b + j]);
  }
  void set_tag(int64_t b, int64_t bits) {
    live[tag[b]] -= 1;
    tag[b] = bits;
    live[bits] += 1;
  }
};

// Plans one step's writes from its slot mapping into the planner's "last plan"
// members; EKH_OK, EKH_EINVAL (a slot past the pool) or EKH_ESLOTS.
int plan_rows(Planner& p, const int64_t* slot_mapping, int64_t n_rows);

// (Re)opens blocks in one pool (ekh_pool_open's work).
int pool_open(Pool& q, const int64_t* blocks, int64_t n, int32_t target_bits, const int64_t* protect,
              int64_t n_protect, uint8_t* headers, int64_t* victims, int64_t* n_victims);

// The device row (slot, block, group, fill, bits, mask) sealing eviction ev.
void seal_row(Pool& q, const int64_t* ev, int64_t* row);

// Records a planned step's touched blocks in the per-block bookkeeping.
void commit(Planner& p, int64_t step, const int64_t* touched, int64_t n_touched);

}  // namespace ekh

// The C ABI's opaque handles (include/echokv_host.h).
struct ekh_planner : ekh::Planner {};
struct ekh_pool : ekh::Pool {};

#endif  // ECHOKV_HOST_STATE_H
