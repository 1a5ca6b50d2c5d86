// The per-step host driver of a KV-cache group (ekh_stepper_*), and the host
// slot mapping (ekh_host_slots). Declared in include/echokv_host.h.
//
// One ekh_stepper_run call does everything a step decides on the host, for
// every layer of the group, and writes the result as one int64 image that the
// caller copies to the device in one transfer:
//   * the batch layout: decode entries (one per single-token request; every
//     request of a decode-only batch, graph padding included), prefill entries,
//     and the canary's query rows on a fire step;
//   * the write plan (plan_rows in plan.cpp);
//   * the blocks that open this step, opened in every layer's pool at that
//     layer's tier, with their page headers and any demotion victims;
//   * the seal rows of evicted residual groups, per layer.
// The graph-visible parts (counts, canary rows, decode entries, token rows, fin
// rows) sit at offsets fixed by the capacity, so a HIP graph captured at any
// batch size up to the capacity reads the current step. The rest (residual map,
// opened ids, headers, seal rows) follows and is consumed by launches the
// builder makes outside any graph.
#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "echokv_host.h"
#include "state.h"

namespace {

struct Stepper {
  ekh::Planner* p = nullptr;
  std::vector<ekh::Pool*> pools;
  int64_t cap = 0;
  int32_t nq = 0;
  // Outputs of the last run, valid until the next.
  std::vector<int64_t> prefill, victims, image;
  // Scratch.
  std::vector<int64_t> dec_row, dec_req, dec_len, opens, protect, seal, hdr, vict;
  std::vector<uint8_t> hdr_bytes;
};

inline int64_t even(int64_t x) { return x + (x & 1); }

}  // namespace

struct ekh_stepper : Stepper {};

extern "C" {

ekh_stepper* ekh_stepper_new(ekh_planner* planner, ekh_pool* const* pools, int32_t n_layers, int64_t cap,
                             int32_t canary_slots) {
  if (!planner || planner->growable || !pools || n_layers <= 0 || cap <= 0 || canary_slots < 0) return nullptr;
  for (int32_t l = 0; l < n_layers; ++l)
    if (!pools[l] || pools[l]->p != planner) return nullptr;
  ekh_stepper* s = new (std::nothrow) ekh_stepper();
  if (!s) return nullptr;
  s->p = planner;
  s->pools.assign(pools, pools + n_layers);
  s->cap = even(cap);
  s->nq = canary_slots;
  s->vict.resize(planner->nb);
  return s;
}

void ekh_stepper_free(ekh_stepper* s) { delete s; }

int ekh_stepper_run(ekh_stepper* S, const ekh_batch* b, const int32_t* tiers, int32_t fire, int64_t* image,
                    int64_t image_cap, ekh_step_view* out) {
  if (!S || !b || !tiers || !out || b->num_reqs < 0 || b->num_tokens < 0) return EKH_EINVAL;
  if (b->num_reqs && (!b->query_start || !b->seq_lens)) return EKH_EINVAL;
  if (b->num_tokens && !b->slot_mapping) return EKH_EINVAL;
  Stepper& s = *S;
  ekh::Planner& p = *s.p;
  const int64_t n = b->num_reqs, t = b->num_tokens;
  const int32_t* qs = b->query_start;
  const int32_t* lens = b->seq_lens;
  const int nlay = (int)s.pools.size();
  for (int l = 0; l < nlay; ++l)
    if (tiers[l] != 2 && tiers[l] != 4 && tiers[l] != 8) return EKH_EINVAL;
  for (int64_t r = 0; r < n; ++r)
    if (qs[r] < 0 || qs[r + 1] < qs[r] || qs[r + 1] > t || lens[r] < 0) return EKH_EINVAL;

  // The batch layout. A request with no query tokens or an empty sequence takes
  // no part; single-token requests decode, longer ones prefill. In a batch with
  // no prefill (what a graph replays) every request is a decode entry, and the
  // padding requests carry length 0.
  bool decode_only = true;
  for (int64_t r = 0; r < n && decode_only; ++r) decode_only = qs[r + 1] - qs[r] <= 1;
  s.dec_row.clear();
  s.dec_req.clear();
  s.dec_len.clear();
  s.prefill.clear();
  int64_t n_canary = 0;
  double ctx_sum = 0.0;
  std::vector<int64_t> canary(s.nq, 0);
  for (int64_t r = 0; r < n; ++r) {
    const int64_t q0 = qs[r], ql = qs[r + 1] - qs[r];
    const bool live = ql > 0 && lens[r] > 0;
    if (decode_only || (live && ql == 1)) {
      s.dec_row.push_back(std::min<int64_t>(q0, std::max<int64_t>(t - 1, 0)));
      s.dec_req.push_back(r);
      s.dec_len.push_back(ql == 1 ? lens[r] : 0);
    } else if (live) {
      s.prefill.insert(s.prefill.end(), {q0, q0 + ql, (int64_t)lens[r], r});
    }
    if (fire && live && n_canary < s.nq) {  // the newest row of the first live requests
      canary[n_canary++] = q0 + ql - 1;
      ctx_sum += lens[r];
    }
  }

  // The write plan, then the blocks that open: offset-0 writes, and writes into
  // blocks no layer has opened yet (the same blocks in every layer).
  const int rc = ekh::plan_rows(p, b->slot_mapping, t);
  if (rc != EKH_OK) return rc;
  const int64_t n_touch = (int64_t)p.touched.size() / 3;
  s.protect.resize(n_touch);
  s.opens = p.opens;
  const ekh::Pool& first = *s.pools[0];
  for (int64_t i = 0; i < n_touch; ++i) {
    const int64_t blk = p.touched[3 * i];
    s.protect[i] = blk;
    if (first.tag[blk] == 0) s.opens.push_back(blk);
  }
  std::sort(s.opens.begin(), s.opens.end());
  s.opens.erase(std::unique(s.opens.begin(), s.opens.end()), s.opens.end());
  const int64_t n_open = (int64_t)s.opens.size();

  // Evicted groups that hold tokens are sealed in every layer, before the slot
  // is reused; then every layer opens the blocks at its own tier.
  int64_t n_seal = 0;
  for (size_t e = 0; e < p.evict.size(); e += 4) n_seal += p.evict[e + 3] > 0;
  s.seal.resize(6 * n_seal * nlay);
  s.hdr_bytes.resize(16 * n_open * nlay);
  s.victims.clear();
  for (int l = 0; l < nlay; ++l) {
    ekh::Pool& q = *s.pools[l];
    int64_t k = 0;
    for (size_t e = 0; e < p.evict.size(); e += 4)
      if (p.evict[e + 3] > 0) ekh::seal_row(q, &p.evict[e], &s.seal[6 * (l * n_seal + k++)]);
    if (!n_open) continue;
    int64_t nv = 0;
    const int orc = ekh::pool_open(q, s.opens.data(), n_open, tiers[l], s.protect.data(), n_touch,
                                   &s.hdr_bytes[16 * n_open * l], s.vict.data(), &nv);
    if (orc != EKH_OK) return orc;  // blocks come from the plan: cannot fail past its checks
    for (int64_t i = 0; i < nv; ++i) s.victims.insert(s.victims.end(), {(int64_t)l, s.vict[i]});
  }
  ekh::commit(p, p.step, p.touched.data(), n_touch);

  // The image.
  const int64_t n_dec = (int64_t)s.dec_row.size(), w = 3 + p.kg;
  const bool fits = n_dec <= s.cap && t <= s.cap && p.n_fin <= s.cap;
  const int64_t r_dec = fits ? s.cap : even(n_dec), r_tok = fits ? s.cap : even(t),
                r_fin = fits ? s.cap : even(p.n_fin);
  const int64_t n_res = (int64_t)p.res_b.size(), n_grp = (int64_t)p.grp_s.size();
  ekh_step_view& v = *out;
  v.step = p.step;
  v.o_canary = 2;
  v.o_mask = v.o_canary + even(s.nq);
  v.o_dec = v.o_mask + even(nlay);
  v.o_tok = v.o_dec + 3 * r_dec;
  v.o_fin = v.o_tok + 4 * r_tok;
  v.o_res = v.o_fin + r_fin * w;
  v.o_grp = v.o_res + 2 * n_res;
  v.o_open = v.o_grp + 2 * n_grp;
  v.o_hdr = v.o_open + n_open;
  v.o_seal = v.o_hdr + 2 * n_open * nlay;
  v.len = v.o_seal + 6 * n_seal * nlay;
  v.rows_dec = r_dec;
  v.rows_tok = r_tok;
  v.rows_fin = r_fin;
  v.n_dec = n_dec;
  v.n_tokens = t;
  v.n_fin = p.n_fin;
  v.n_res = n_res;
  v.n_grp = n_grp;
  v.n_open = n_open;
  v.n_seal = n_seal;
  v.n_canary = n_canary;
  v.decode_only = decode_only;
  v.canary_ctx = n_canary ? ctx_sum / (double)n_canary : 0.0;
  v.n_prefill = (int64_t)s.prefill.size() / 4;
  v.prefill = s.prefill.data();
  v.n_victims = (int64_t)s.victims.size() / 2;
  v.victims = s.victims.data();
  v.graph_rows = fits;

  int64_t* img = image;
  if (!img || v.len > image_cap) {  // a step larger than the caller's buffer: the stepper's own
    s.image.assign(v.len, 0);
    img = s.image.data();
  }
  v.image = img;
  img[0] = p.n_fin;
  img[1] = t;
  std::copy(canary.begin(), canary.end(), img + v.o_canary);
  // Each layer's tiers with live blocks (2 | 4 | 8), after this step's opens: the
  // decode kernels read it to run each present tier's blocks on its own path.
  for (int l = 0; l < nlay; ++l) {
    const int64_t* live = s.pools[l]->live;
    img[v.o_mask + l] = (live[2] ? 2 : 0) | (live[4] ? 4 : 0) | (live[8] ? 8 : 0);
  }
  std::copy(s.dec_row.begin(), s.dec_row.end(), img + v.o_dec);
  std::copy(s.dec_req.begin(), s.dec_req.end(), img + v.o_dec + r_dec);
  std::copy(s.dec_len.begin(), s.dec_len.end(), img + v.o_dec + 2 * r_dec);
  if (t) std::copy(b->slot_mapping, b->slot_mapping + t, img + v.o_tok);
  std::copy(p.tok_res.begin(), p.tok_res.end(), img + v.o_tok + r_tok);
  std::copy(p.tok_sealed.begin(), p.tok_sealed.end(), img + v.o_tok + 2 * r_tok);
  std::copy(p.tok_kref.begin(), p.tok_kref.end(), img + v.o_tok + 3 * r_tok);
  std::copy(p.fin.begin(), p.fin.end(), img + v.o_fin);
  int64_t* o = img + v.o_res;
  o = std::copy(p.res_b.begin(), p.res_b.end(), o);
  o = std::copy(p.res_v.begin(), p.res_v.end(), o);
  o = std::copy(p.grp_s.begin(), p.grp_s.end(), o);
  o = std::copy(p.grp_g.begin(), p.grp_g.end(), o);
  o = std::copy(s.opens.begin(), s.opens.end(), o);
  if (n_open) std::memcpy(o, s.hdr_bytes.data(), s.hdr_bytes.size());
  o += 2 * n_open * nlay;
  std::copy(s.seal.begin(), s.seal.end(), o);
  return EKH_OK;
}

int ekh_host_slots(const ekh_batch* b, const int32_t* table, int64_t table_rows, int64_t table_cols,
                   int64_t table_stride, const int64_t* row_map, int64_t row_map_len, int32_t block_size,
                   int64_t* slots) {
  if (!b || !table || !slots || block_size <= 0 || b->num_reqs < 0 || b->num_tokens < 0) return EKH_EINVAL;
  if (b->num_reqs && (!b->query_start || !b->seq_lens)) return EKH_EINVAL;
  const int32_t* qs = b->query_start;
  const int64_t n = b->num_reqs;
  if (n && qs[n] > b->num_tokens) return EKH_EINVAL;
  int64_t done = 0;
  for (int64_t r = 0; r < n; ++r) {
    const int64_t q0 = qs[r], q1 = qs[r + 1];
    if (q0 != done || q1 < q0) return EKH_EINVAL;
    const int64_t row = row_map ? (r < row_map_len ? row_map[r] : -1) : r;
    if (q1 > q0 && (row < 0 || row >= table_rows)) return EKH_EINVAL;
    const int64_t first = (int64_t)b->seq_lens[r] - (q1 - q0);  // position of the request's first query token
    if (first < 0) return EKH_EINVAL;
    const int32_t* tr = table + row * table_stride;
    for (int64_t i = q0; i < q1; ++i) {
      const int64_t pos = first + (i - q0), col = pos / block_size;
      if (col >= table_cols) return EKH_EINVAL;
      slots[i] = (int64_t)tr[col] * block_size + pos % block_size;
    }
    done = q1;
  }
  for (int64_t i = done; i < b->num_tokens; ++i) slots[i] = -1;  // padding rows write nothing
  return EKH_OK;
}

}  // extern "C"
