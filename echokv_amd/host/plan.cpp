// Native host side of the tiered KV store: the per-step write planner shared by
// every layer of a KV-cache group, and each layer's chunk pool. Plain C++17 on
// the CPU (no HIP), bound from Python with ctypes; declared in
// include/echokv_host.h.
//
// The decisions are the reference's (they decide which bytes land where, and the
// golden page bytes pin them):
//   * residual slots: a LIFO stack (slot 0 handed out first, a released slot
//     next); when none is free, the least recently written slot not mapped by a
//     block of this step is evicted (ties: the slot taken earliest), and its
//     group is sealed (echokv_vllm/write_plan.py:98-240);
//   * a (block, K group) whose K-group tokens are all in the step is finalized
//     from the key rows; a group completing from the residual is finalized with
//     its slot; others go to the residual (or under sealed stats);
//   * chunk pool: a stack of chunk ids page * KC + slot (slots >= 1), lowest id
//     first; blocks open greedily in block order (INT8 while chunks last, then
//     INT4, then INT2); when short, least recently written full INT4 / INT8 blocks
//     are demoted (ties: lowest block id) (echokv_vllm/tiered_cache.py:196-347).
// The implementation is this build's: dense per-block arrays instead of hash
// maps, a step stamp for the protected set, one sort of the step's tokens, and
// the plan written straight into the staging image the device reads.
#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "echokv_host.h"
#include "state.h"

namespace ekh {

void Planner::grow(int64_t need) {
  if (need <= nb) return;
  const int64_t n = std::max<int64_t>(need, 2 * nb);
  block_slot.resize(n, -1);
  sealed.resize(n, 0);
  fill_h.resize(n, 0);
  last_h.resize(n, 0);
  cum_h.resize(n, 0);
  res_stamp.resize(n, 0);
  res_at.resize(n, 0);
  nb = n;
}

void Planner::res_op(int64_t b, int64_t v) {
  if (res_stamp[b] == step) {
    res_v[res_at[b]] = v;
  } else {
    res_stamp[b] = step;
    res_at[b] = (int64_t)res_b.size();
    res_b.push_back(b);
    res_v.push_back(v);
  }
}

void Planner::grp_op(int32_t s, int32_t g) {
  if (grp_stamp[s] == step) {
    grp_g[grp_at[s]] = g;
  } else {
    grp_stamp[s] = step;
    grp_at[s] = (int64_t)grp_s.size();
    grp_s.push_back(s);
    grp_g.push_back(g);
  }
}

void Planner::release(int32_t s) {
  const int64_t b = s_block[s];
  s_used[s] = 0;
  block_slot[b] = -1;
  free_stack.push_back(s);
  res_op(b, -1);
}

// The least recently written slot outside this step's protected set, or -1.
int32_t Planner::victim() const {
  int32_t best = -1;
  for (int32_t s = 0; s < R; ++s) {
    if (!s_used[s] || s_prot[s] == step) continue;
    if (best < 0 || s_last[s] < s_last[best] || (s_last[s] == s_last[best] && s_taken[s] < s_taken[best])) best = s;
  }
  return best;
}

int32_t Planner::take(int64_t b, int32_t g) {
  const int32_t s = free_stack.back();
  free_stack.pop_back();
  s_used[s] = 1;
  s_block[s] = b;
  s_group[s] = g;
  s_fill[s] = 0;
  s_last[s] = 0;
  s_taken[s] = ++taken;
  s_prot[s] = step;
  block_slot[b] = s;
  res_op(b, s);
  grp_op(s, g);
  return s;
}

}  // namespace ekh

using ekh::kExtra;
using ekh::Planner;
using ekh::Pool;

namespace ekh {

int plan_rows(Planner& p, const int64_t* slot_mapping, int64_t n_rows) {
  int64_t top_slot = -1;
  for (int64_t r = 0; r < n_rows; ++r) top_slot = std::max(top_slot, slot_mapping[r]);
  if (top_slot >= p.nb * p.bs) {
    if (!p.growable) return EKH_EINVAL;  // a slot past the last block
    p.grow(top_slot / p.bs + 1);
  }
  const int bs = p.bs, kg = p.kg, gpb = p.gpb;
  p.step += 1;
  p.n_rows = n_rows;
  p.evict.clear();
  p.opens.clear();
  p.touched.clear();
  p.res_b.clear();
  p.res_v.clear();
  p.grp_s.clear();
  p.grp_g.clear();

  // Token rows that write (slot >= 0), their (block, K group) keys, sorted by
  // key, then position in the group, then row (so equal slots keep row order).
  p.rows.clear();
  for (int64_t r = 0; r < n_rows; ++r)
    if (slot_mapping[r] >= 0) p.rows.push_back(r);
  const int64_t n = (int64_t)p.rows.size();
  p.key.resize(n);
  p.order.resize(n);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t s = slot_mapping[p.rows[i]];
    p.key[i] = (s / bs) * gpb + (s % bs) / kg;
    p.order[i] = i;
  }
  auto pos_of = [&](int64_t i) { return (slot_mapping[p.rows[i]] % bs) % kg; };
  std::sort(p.order.begin(), p.order.end(), [&](int64_t a, int64_t b) {
    if (p.key[a] != p.key[b]) return p.key[a] < p.key[b];
    const int64_t pa = pos_of(a), pb = pos_of(b);
    return pa != pb ? pa < pb : a < b;
  });

  // Blocks (re)opened this step (an offset-0 write), ascending: their open group
  // leaves the residual and their sealed marks reset.
  for (int64_t i = 0; i < n; ++i) {
    const int64_t s = slot_mapping[p.rows[p.order[i]]];
    if (s % bs == 0 && (p.opens.empty() || p.opens.back() != s / bs)) p.opens.push_back(s / bs);
  }
  for (int64_t b : p.opens) {
    if (p.block_slot[b] >= 0) p.release(p.block_slot[b]);
    p.sealed[b] = 0;
  }

  // Runs of equal key = the step's (block, group) units, in key order.
  struct Unit {
    int64_t start, count, blk;
    int32_t grp;
    bool whole;
  };
  std::vector<Unit> units;
  for (int64_t i = 0; i < n;) {
    int64_t j = i + 1;
    while (j < n && p.key[p.order[j]] == p.key[p.order[i]]) ++j;
    const int64_t k = p.key[p.order[i]];
    units.push_back(Unit{i, j - i, k / gpb, (int32_t)(k % gpb), false});
    i = j;
  }
  // Whole groups (all K-group positions in this step, not sealed) finalize from
  // the key rows; a residual slot still holding one of them is released.
  for (size_t u = 0; u < units.size(); ++u) {
    Unit& x = units[u];
    x.whole = x.count == kg && !((p.sealed[x.blk] >> x.grp) & 1);
  }
  for (size_t u = 0; u < units.size();) {  // per block, at its first whole group
    size_t v = u;
    uint32_t mask = 0;
    while (v < units.size() && units[v].blk == units[u].blk) {
      if (units[v].whole) mask |= 1u << units[v].grp;
      ++v;
    }
    const int32_t s = p.block_slot[units[u].blk];
    if (mask && s >= 0 && ((mask >> p.s_group[s]) & 1)) p.release(s);
    u = v;
  }
  // Slots of the step's blocks cannot be evicted by this step.
  for (size_t u = 0; u < units.size(); ++u) {
    const int32_t s = p.block_slot[units[u].blk];
    if (s >= 0) p.s_prot[s] = p.step;
  }

  // Per-row outputs, and the fin rows (whole groups first, then the others).
  const int64_t w = 3 + kg;
  p.tok_res.assign(n_rows, -1);
  p.tok_sealed.assign(n_rows, 0);
  p.tok_kref.assign(n_rows, -1);
  std::vector<int64_t>& tok_res = p.tok_res;
  std::vector<int64_t>& tok_sealed = p.tok_sealed;
  std::vector<int64_t>& tok_kref = p.tok_kref;
  std::vector<int64_t>& fin_whole = p.fin;
  std::vector<int64_t> fin_rest;
  fin_whole.clear();
  for (const Unit& x : units) {
    if (!x.whole) continue;
    fin_whole.push_back(x.blk);
    fin_whole.push_back(x.grp);
    fin_whole.push_back(-1);
    for (int64_t i = 0; i < x.count; ++i) fin_whole.push_back(p.rows[p.order[x.start + i]]);
  }
  for (const Unit& x : units) {
    if (x.whole) continue;
    if ((p.sealed[x.blk] >> x.grp) & 1) {  // quantized under the group's stored stats
      for (int64_t i = 0; i < x.count; ++i) tok_sealed[p.rows[p.order[x.start + i]]] = 1;
      continue;
    }
    int32_t s = p.block_slot[x.blk];
    if (s >= 0 && p.s_group[s] != x.grp) s = -1;  // a slot of another group of the block
    const int64_t top = pos_of(p.order[x.start + x.count - 1]);
    if (top == kg - 1) {  // the group completes now: finalize it (residual positions -1)
      fin_rest.push_back(x.blk);
      fin_rest.push_back(x.grp);
      fin_rest.push_back(s);
      const size_t at = fin_rest.size();
      fin_rest.resize(at + kg, -1);
      for (int64_t i = 0; i < x.count; ++i) {
        const int64_t t = p.order[x.start + i];
        fin_rest[at + pos_of(t)] = p.rows[t];
      }
      if (s >= 0) p.release(s);
      continue;
    }
    if (s < 0) {
      if (p.free_stack.empty()) {
        const int32_t v = p.victim();
        if (v < 0) return EKH_ESLOTS;
        p.evict.push_back(v);
        p.evict.push_back(p.s_block[v]);
        p.evict.push_back(p.s_group[v]);
        p.evict.push_back(p.s_fill[v]);
        p.sealed[p.s_block[v]] |= (uint8_t)(1u << p.s_group[v]);
        p.release(v);
      }
      s = p.take(x.blk, x.grp);
    }
    for (int64_t i = 0; i < x.count; ++i) tok_res[p.rows[p.order[x.start + i]]] = s;
    p.s_fill[s] = std::max<int32_t>(p.s_fill[s], (int32_t)top + 1);
    p.s_last[s] = p.step;
  }

  // Touched blocks (ascending): highest offset written + 1, and token count.
  for (int64_t i = 0; i < n;) {
    const int64_t b = p.key[p.order[i]] / gpb;
    int64_t fill = 0, cnt = 0;
    for (; i < n && p.key[p.order[i]] / gpb == b; ++i) {
      fill = std::max<int64_t>(fill, slot_mapping[p.rows[p.order[i]]] % bs + 1);
      ++cnt;
    }
    p.touched.push_back(b);
    p.touched.push_back(fill);
    p.touched.push_back(cnt);
  }

  // The step's last kref_window keys enter the K_ref ring, in row order.
  const int64_t k = std::min<int64_t>(n, p.W);
  for (int64_t i = 0; i < k; ++i) tok_kref[p.rows[n - k + i]] = (p.kref_pos + i) % p.W;
  p.kref_pos = (p.kref_pos + k) % p.W;
  p.kref_fill = std::min<int64_t>(p.W, p.kref_fill + k);

  p.n_fin = (int64_t)(fin_whole.size() + fin_rest.size()) / w;
  fin_whole.insert(fin_whole.end(), fin_rest.begin(), fin_rest.end());
  return EKH_OK;
}

void commit(Planner& p, int64_t step, const int64_t* touched, int64_t n_touched) {
  for (int64_t i = 0; i < n_touched; ++i) {
    const int64_t b = touched[3 * i];
    p.fill_h[b] = std::max(p.fill_h[b], touched[3 * i + 1]);
    p.last_h[b] = step;
    p.cum_h[b] += touched[3 * i + 2];
  }
}

}  // namespace ekh

namespace ekh {

int pool_open(Pool& q, const int64_t* blocks, int64_t n, int32_t target_bits, const int64_t* protect,
              int64_t n_protect, uint8_t* headers, int64_t* victims, int64_t* n_victims) {
  if (target_bits != 2 && target_bits != 4 && target_bits != 8) return EKH_EINVAL;
  for (int64_t i = 0; i < n; ++i)
    if (blocks[i] < 0 || blocks[i] >= q.nb) return EKH_EINVAL;
  *n_victims = 0;
  for (int64_t i = 0; i < n; ++i) {  // old chunks go back to the pool
    const int64_t b = blocks[i];
    q.settle(b);
    q.give_back(b);
    q.set_tag(b, 0);
  }
  const int64_t need = (int64_t)kExtra[target_bits] * n;
  if (need > (int64_t)q.free_chunks.size()) {
    // Least recently written full INT4 / INT8 blocks, never this step's.
    std::vector<uint8_t> keep(q.nb, 0);
    for (int64_t i = 0; i < n; ++i) keep[blocks[i]] = 1;
    for (int64_t i = 0; i < n_protect; ++i)
      if (protect[i] >= 0 && protect[i] < q.nb) keep[protect[i]] = 1;
    std::vector<int64_t> cand;
    for (int64_t b = 0; b < q.nb; ++b)
      if (q.tag[b] >= 4 && q.p->fill_h[b] == q.bs && !keep[b]) cand.push_back(b);
    std::stable_sort(cand.begin(), cand.end(),
                     [&](int64_t a, int64_t b) { return q.p->last_h[a] < q.p->last_h[b]; });
    const int64_t short_by = need - (int64_t)q.free_chunks.size();
    int64_t freed = 0;
    for (int64_t b : cand) {
      if (freed >= short_by) break;
      victims[(*n_victims)++] = b;
      freed += kExtra[q.tag[b]];
    }
    for (int64_t i = 0; i < *n_victims; ++i) {  // requantized to INT2 on the device by the caller
      const int64_t b = victims[i];
      q.settle(b);
      q.give_back(b);
      q.set_tag(b, 2);
    }
    q.demoted += *n_victims;
  }
  // Greedy in block order: INT8 while it fits, then INT4, then INT2.
  std::vector<int32_t> tiers(n, 2);
  int64_t start = 0;
  for (int bits : {8, 4}) {
    if (bits > target_bits) continue;
    const int ne = kExtra[bits];
    const int64_t take = std::min<int64_t>(n - start, (int64_t)q.free_chunks.size() / ne);
    for (int64_t i = start; i < start + take; ++i) {
      for (int j = 0; j < ne; ++j) {
        q.table[3 * blocks[i] + j] = q.free_chunks.back();
        q.free_chunks.pop_back();
      }
      tiers[i] = bits;
    }
    start += take;
  }
  for (int64_t i = 0; i < n; ++i) {
    const int64_t b = blocks[i];
    q.opened[tiers[i]] += 1;
    if (tiers[i] < target_bits) q.downgraded += 1;
    q.set_tag(b, tiers[i]);
    uint8_t* h = headers + 16 * i;
    std::memset(h, 0, 16);
    h[0] = (uint8_t)tiers[i];
    for (int j = 0; j < 3; ++j) {
      const int32_t id = (int32_t)q.table[3 * b + j];
      std::memcpy(h + 4 + 4 * j, &id, 4);
    }
  }
  return EKH_OK;
}


}  // namespace ekh

namespace ekh {

void seal_row(Pool& q, const int64_t* ev, int64_t* row) {
  // ev = (slot, block, group, fill) -> device row (slot, block, group, fill, bits, mask)
  const int64_t b = ev[1];
  q.sealed_groups += 1;
  const int32_t mask = q.p->sealed[b];
  row[0] = ev[0];
  row[1] = b;
  row[2] = ev[2];
  row[3] = ev[3];
  row[4] = q.tag[b] ? q.tag[b] : 2;
  row[5] = mask ? mask : (1 << ev[2]);
}

}  // namespace ekh


extern "C" {

ekh_planner* ekh_planner_new(int64_t num_blocks, int32_t block_size, int32_t k_group, int32_t residual_slots,
                             int32_t kref_window) {
  if (block_size <= 0 || k_group <= 0 || block_size % k_group || block_size / k_group > 8 || residual_slots <= 0 ||
      kref_window <= 0)
    return nullptr;
  ekh_planner* p = new (std::nothrow) ekh_planner();
  if (!p) return nullptr;
  p->growable = num_blocks <= 0;
  if (p->growable) num_blocks = 1;
  p->nb = num_blocks;
  p->bs = block_size;
  p->kg = k_group;
  p->gpb = block_size / k_group;
  p->R = residual_slots;
  p->W = kref_window;
  for (int32_t s = residual_slots - 1; s >= 0; --s) p->free_stack.push_back(s);
  p->s_block.assign(residual_slots, -1);
  p->s_last.assign(residual_slots, 0);
  p->s_taken.assign(residual_slots, 0);
  p->s_prot.assign(residual_slots, 0);
  p->s_group.assign(residual_slots, 0);
  p->s_fill.assign(residual_slots, 0);
  p->s_used.assign(residual_slots, 0);
  p->grp_stamp.assign(residual_slots, 0);
  p->grp_at.assign(residual_slots, 0);
  p->block_slot.assign(num_blocks, -1);
  p->sealed.assign(num_blocks, 0);
  p->fill_h.assign(num_blocks, 0);
  p->last_h.assign(num_blocks, 0);
  p->cum_h.assign(num_blocks, 0);
  p->res_stamp.assign(num_blocks, 0);
  p->res_at.assign(num_blocks, 0);
  return p;
}

void ekh_planner_free(ekh_planner* p) { delete p; }

int ekh_plan(ekh_planner* P, const int64_t* slot_mapping, int64_t n_rows, ekh_plan_view* out) {
  if (!P || !out || n_rows < 0 || (n_rows && !slot_mapping)) return EKH_EINVAL;
  Planner& p = *P;
  const int rc = ekh::plan_rows(p, slot_mapping, n_rows);
  if (rc != EKH_OK) return rc;
  // The staging image: one contiguous int64 buffer, copied to the device as is.
  const int64_t nres = (int64_t)p.res_b.size(), ngrp = (int64_t)p.grp_s.size();
  p.stage.assign(1 + 4 * n_rows + (int64_t)p.fin.size() + 2 * nres + 2 * ngrp, 0);
  int64_t* o = p.stage.data();
  *o++ = p.n_fin;
  o = std::copy(slot_mapping, slot_mapping + n_rows, o);
  o = std::copy(p.tok_res.begin(), p.tok_res.end(), o);
  o = std::copy(p.tok_sealed.begin(), p.tok_sealed.end(), o);
  o = std::copy(p.tok_kref.begin(), p.tok_kref.end(), o);
  o = std::copy(p.fin.begin(), p.fin.end(), o);
  o = std::copy(p.res_b.begin(), p.res_b.end(), o);
  o = std::copy(p.res_v.begin(), p.res_v.end(), o);
  o = std::copy(p.grp_s.begin(), p.grp_s.end(), o);
  std::copy(p.grp_g.begin(), p.grp_g.end(), o);

  out->step = p.step;
  out->n_rows = n_rows;
  out->n_fin = p.n_fin;
  out->n_evict = (int64_t)p.evict.size() / 4;
  out->n_open = (int64_t)p.opens.size();
  out->n_touched = (int64_t)p.touched.size() / 3;
  out->n_res_map = nres;
  out->n_grp_map = ngrp;
  out->stage = p.stage.data();
  out->stage_len = (int64_t)p.stage.size();
  out->evict = p.evict.data();
  out->open = p.opens.data();
  out->touched = p.touched.data();
  return EKH_OK;
}

int ekh_commit(ekh_planner* p, int64_t step, const int64_t* touched, int64_t n_touched) {
  for (int64_t i = 0; i < n_touched; ++i)
    if (touched[3 * i] < 0 || touched[3 * i] >= p->nb) return EKH_EINVAL;
  ekh::commit(*p, step, touched, n_touched);
  return EKH_OK;
}

int64_t ekh_planner_state(const ekh_planner* p, int32_t what) {
  switch (what) {
    case EKH_STEP: return p->step;
    case EKH_RES_FREE: return (int64_t)p->free_stack.size();
    case EKH_RES_SLOTS: return p->R;
    case EKH_KREF_POS: return p->kref_pos;
    case EKH_KREF_FILL: return p->kref_fill;
    case EKH_KREF_WINDOW: return p->W;
    case EKH_NUM_BLOCKS: return p->nb;
    default: return -1;
  }
}

int64_t ekh_residual_free_list(const ekh_planner* p, int64_t* out, int64_t cap) {
  const int64_t n = (int64_t)p->free_stack.size();
  for (int64_t i = 0; i < n && i < cap; ++i) out[i] = p->free_stack[i];
  return n;
}

int32_t ekh_sealed_mask(const ekh_planner* p, int64_t block) {
  return block >= 0 && block < p->nb ? p->sealed[block] : 0;
}

int64_t* ekh_block_array(ekh_planner* p, int32_t which) {
  switch (which) {
    case EKH_FILL: return p->fill_h.data();
    case EKH_LAST: return p->last_h.data();
    case EKH_CUM: return p->cum_h.data();
    default: return nullptr;
  }
}

// ---- chunk pool ------------------------------------------------------------

ekh_pool* ekh_pool_new(ekh_planner* planner, int32_t chunks_per_page) {
  if (!planner || planner->growable || chunks_per_page < 1 || chunks_per_page > 4) return nullptr;
  ekh_pool* q = new (std::nothrow) ekh_pool();
  if (!q) return nullptr;
  q->p = planner;
  q->nb = planner->nb;
  q->kc = chunks_per_page;
  q->bs = planner->bs;
  for (int64_t page = q->nb - 1; page >= 0; --page)
    for (int slot = chunks_per_page - 1; slot >= 1; --slot) q->free_chunks.push_back(page * chunks_per_page + slot);
  q->pool_size = (int64_t)q->free_chunks.size();
  q->tag.assign(q->nb, 0);
  q->live[0] = q->nb;
  q->table.assign(3 * q->nb, 0);
  q->mark = planner->cum_h;
  return q;
}

void ekh_pool_free(ekh_pool* q) { delete q; }

int ekh_pool_open(ekh_pool* Q, const int64_t* blocks, int64_t n, int32_t target_bits, const int64_t* protect,
                  int64_t n_protect, uint8_t* headers, int64_t* victims, int64_t* n_victims) {
  if (!Q || n < 0 || (n && (!blocks || !headers)) || !victims || !n_victims) return EKH_EINVAL;
  return ekh::pool_open(*Q, blocks, n, target_bits, protect, n_protect, headers, victims, n_victims);
}

int64_t ekh_pool_seal_row(ekh_pool* q, const int64_t* ev, int64_t* row) {
  if (ev[1] < 0 || ev[1] >= q->nb) return EKH_EINVAL;
  ekh::seal_row(*q, ev, row);
  return EKH_OK;
}

void ekh_pool_counters(const ekh_pool* q, int64_t* out) {
  // out[0..8]: tokens written per tier (settled + pending), out[9..17]: blocks
  // opened per tier, then downgraded, demoted, sealed groups, free chunks, pool size.
  for (int b = 0; b < 9; ++b) out[b] = q->tok_tier[b];
  for (int64_t i = 0; i < q->nb; ++i) out[q->tag[i]] += q->p->cum_h[i] - q->mark[i];
  for (int b = 0; b < 9; ++b) out[9 + b] = q->opened[b];
  out[18] = q->downgraded;
  out[19] = q->demoted;
  out[20] = q->sealed_groups;
  out[21] = (int64_t)q->free_chunks.size();
  out[22] = q->pool_size;
}

void ekh_pool_reset_counters(ekh_pool* q) {
  std::fill(q->tok_tier, q->tok_tier + 9, 0);
  q->mark = q->p->cum_h;
  std::fill(q->opened, q->opened + 9, 0);
  q->downgraded = q->demoted = q->sealed_groups = 0;
}

int64_t* ekh_pool_tags(ekh_pool* q) { return q->tag.data(); }

void ekh_pool_live(const ekh_pool* q, int64_t* out) { std::copy(q->live, q->live + 9, out); }

int64_t ekh_pool_free_list(const ekh_pool* q, int64_t* out, int64_t cap) {
  const int64_t n = (int64_t)q->free_chunks.size();
  for (int64_t i = 0; i < n && i < cap; ++i) out[i] = q->free_chunks[i];
  return n;
}

}  // extern "C"
