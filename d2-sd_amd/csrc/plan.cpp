// Host-side work planning for cascade verify attention (plan()).
//
// Splits every request's visible prefix into key chunks (split-KV) so that the
// attention launch fills the device, adds one suffix (tree) item per q-tile,
// and orders the work list so that all q-tiles reading one key chunk are dealt
// to the same XCD.  No reference counterpart: FlashInfer's planner is not in
// the reference tree; the reference only ever issues one un-split
// single_prefill per level (generation/verification.py:145, 159).
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <vector>

#include "d2sd_internal.h"
#include "plan.h"

namespace d2sd {

namespace {

struct KvSet {  // all q-tiles of one (request, kv head) reading one key range
  int req, kvh, src, kv_begin, kv_end, qtiles;
  long long cost;  // tiles * qtiles
  int first_slot_of_qtile0;
};

}  // namespace

int choose_waves(int rows_per_head_max) {
  // 8 waves (256 rows) once a head has more than 128 packed rows; a 4-wave
  // tile otherwise, so that small problems do not idle half a workgroup.
  return rows_per_head_max > 128 ? 8 : 4;
}

int blocks_per_cu(int waves) { return waves == 4 ? 2 : 1; }

int plan_cascade(const PlanInput& in, std::vector<WorkItem>& work, std::vector<MergeItem>& merge,
                 PlanOutput& out) {
  work.clear();
  merge.clear();
  const int Hkv = in.num_kv_heads;
  const int g = in.num_qo_heads / Hkv;
  int max_rows = 0;
  for (int r = 0; r < in.num_reqs; ++r) max_rows = std::max(max_rows, (in.qo_indptr[r + 1] - in.qo_indptr[r]) * g);
  const int W = in.waves ? in.waves : choose_waves(max_rows);
  const int ROWS = 32 * W;
  const int num_cus = in.num_cus > 0 ? in.num_cus : 256;
  const long long target = (long long)num_cus * blocks_per_cu(W);

  // Groups = (request, kv head, q-tile).
  long long groups = 0, prefix_cost = 0;
  std::vector<int> qtiles(in.num_reqs), ptiles(in.num_reqs), kv0(in.num_reqs), kv1(in.num_reqs);
  for (int r = 0; r < in.num_reqs; ++r) {
    const int nq = in.qo_indptr[r + 1] - in.qo_indptr[r];
    qtiles[r] = (nq * g + ROWS - 1) / ROWS;
    const int L = in.prefix_len[r];
    const int Leff = in.window_left >= 0 ? std::min(L, in.window_left) : L;
    kv0[r] = L - Leff;
    kv1[r] = L;
    ptiles[r] = (Leff + 63) / 64;
    groups += (long long)Hkv * qtiles[r];
    prefix_cost += (long long)Hkv * qtiles[r] * ptiles[r];
  }
  // Key tiles per prefix split: spread the prefix over what the suffix items
  // leave of one wave of workgroups, but never below kMinChunkTiles.
  const int kMinChunkTiles = 2;
  long long avail = std::max<long long>(target - groups, groups);
  long long chunk = std::max<long long>(kMinChunkTiles, (prefix_cost + avail - 1) / std::max<long long>(avail, 1));

  std::vector<KvSet> sets;
  int slot = 0, max_splits_used = 0;
  // slot bookkeeping per group: slot_begin[group], nitems[group]
  std::vector<int> grp_slot_begin, grp_items;
  std::vector<int> grp_req, grp_kvh, grp_qt;
  std::vector<int> req_grp0(in.num_reqs);
  for (int r = 0; r < in.num_reqs; ++r) {
    const int nq = in.qo_indptr[r + 1] - in.qo_indptr[r];
    if (nq == 0) continue;
    int splits = ptiles[r] == 0 ? 0 : (int)((ptiles[r] + chunk - 1) / chunk);
    if (in.max_splits > 0) splits = std::min(splits, in.max_splits);
    max_splits_used = std::max(max_splits_used, splits);
    const int nitems = splits + 1;  // + suffix level
    req_grp0[r] = (int)grp_req.size();
    for (int h = 0; h < Hkv; ++h)
      for (int qt = 0; qt < qtiles[r]; ++qt) {
        grp_req.push_back(r);
        grp_kvh.push_back(h);
        grp_qt.push_back(qt);
        grp_items.push_back(nitems);
        grp_slot_begin.push_back(nitems > 1 ? slot : -1);
        if (nitems > 1) slot += nitems;
      }
    // prefix sets: balanced chunks
    for (int h = 0; h < Hkv; ++h) {
      for (int s = 0; s < splits; ++s) {
        const int base = ptiles[r] / splits, rem = ptiles[r] % splits;
        const int t0 = s * base + std::min(s, rem);
        const int nt = base + (s < rem ? 1 : 0);
        KvSet ks;
        ks.req = r;
        ks.kvh = h;
        ks.src = 0;
        ks.kv_begin = kv0[r] + 64 * t0;
        ks.kv_end = std::min(kv1[r], kv0[r] + 64 * (t0 + nt));
        ks.qtiles = qtiles[r];
        ks.cost = (long long)nt * qtiles[r];
        ks.first_slot_of_qtile0 = s;  // item index inside the group
        sets.push_back(ks);
      }
      KvSet ks;
      ks.req = r;
      ks.kvh = h;
      ks.src = 1;
      ks.kv_begin = 0;
      ks.kv_end = nq;
      ks.qtiles = qtiles[r];
      ks.cost = (long long)((nq + 63) / 64) * qtiles[r];
      ks.first_slot_of_qtile0 = splits;  // suffix is the last item of its group
      sets.push_back(ks);
    }
  }

  // XCD placement: largest sets first onto the least-loaded XCD.
  std::vector<int> order(sets.size());
  for (size_t i = 0; i < sets.size(); ++i) order[i] = (int)i;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return sets[a].cost > sets[b].cost; });
  std::vector<long long> load(8, 0);
  std::vector<std::vector<WorkItem>> lists(8);
  for (int si : order) {
    const KvSet& ks = sets[si];
    int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    load[x] += ks.cost;
    for (int qt = 0; qt < ks.qtiles; ++qt) {
      const int gi = req_grp0[ks.req] + ks.kvh * qtiles[ks.req] + qt;
      WorkItem w;
      w.req = ks.req;
      w.kvh = ks.kvh;
      w.qtile = qt;
      w.src = ks.src;
      w.kv_begin = ks.kv_begin;
      w.kv_end = ks.kv_end;
      if (grp_items[gi] > 1) {
        w.slot = grp_slot_begin[gi] + ks.first_slot_of_qtile0;
        w.mode = MODE_PARTIAL;
      } else {
        w.slot = -1;
        w.mode = MODE_FINAL;
      }
      lists[x].push_back(w);
    }
  }
  size_t maxlen = 0;
  for (auto& l : lists) maxlen = std::max(maxlen, l.size());
  for (size_t k = 0; k < maxlen; ++k)
    for (int x = 0; x < 8; ++x) {
      if (k < lists[x].size()) {
        work.push_back(lists[x][k]);
      } else {
        WorkItem w{};
        w.mode = MODE_NOOP;
        work.push_back(w);
      }
    }
  // Trim trailing padding (never changes the XCD of earlier items).
  while (!work.empty() && work.back().mode == MODE_NOOP) work.pop_back();

  for (size_t gi = 0; gi < grp_req.size(); ++gi) {
    if (grp_items[gi] <= 1) continue;
    MergeItem m{};
    m.req = grp_req[gi];
    m.kvh = grp_kvh[gi];
    m.qtile = grp_qt[gi];
    m.slot_begin = grp_slot_begin[gi];
    m.nslots = grp_items[gi];
    m.mode = MODE_FINAL;
    merge.push_back(m);
  }

  out.waves = W;
  out.rows_per_tile = ROWS;
  out.num_slots = slot;
  out.max_splits_used = max_splits_used;
  out.workspace_bytes = (size_t)slot * ROWS * ((size_t)in.head_dim + 1) * sizeof(float);
  return 0;
}

void plan_single(int qo_len, int kv_len, int num_qo_heads, int num_kv_heads, int head_dim,
                 int window_left, int num_cus, ImplicitWork& imp, int& waves, size_t& workspace_bytes) {
  const int g = num_qo_heads / num_kv_heads;
  const int rows = qo_len * g;
  waves = choose_waves(rows);
  const int ROWS = 32 * waves;
  const int kb = (window_left >= 0 && kv_len > window_left) ? kv_len - window_left : 0;
  const int keys = kv_len - kb;
  const int ntiles = (keys + 63) / 64;
  imp.num_reqs = 1;
  imp.qtiles = std::max(1, (rows + ROWS - 1) / ROWS);
  imp.qo_len = qo_len;
  imp.kv_len = kv_len;
  imp.kv_begin = kb;
  const long long target = (long long)(num_cus > 0 ? num_cus : 256) * blocks_per_cu(waves);
  const long long groups = (long long)num_kv_heads * imp.qtiles;
  int splits = (int)std::max<long long>(1, target / std::max<long long>(groups, 1));
  const int kMinChunkTiles = 2;
  splits = std::min(splits, std::max(1, ntiles / kMinChunkTiles));
  const int chunk_tiles = std::max(1, (ntiles + splits - 1) / splits);
  splits = std::max(1, (ntiles + chunk_tiles - 1) / chunk_tiles);
  imp.splits = splits;
  imp.chunk_keys = 64 * chunk_tiles;
  imp.single_mode = MODE_FINAL;
  workspace_bytes =
      splits > 1 ? (size_t)groups * splits * ROWS * ((size_t)head_dim + 1) * sizeof(float) : 0;
}

}  // namespace d2sd
