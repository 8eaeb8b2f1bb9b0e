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


int choose_waves(int rows_per_head_max) {
  // 8 waves (256 rows) once a head has more than 128 packed rows; a 4-wave
  // tile otherwise, so that small problems do not idle half a workgroup.
  return rows_per_head_max > 128 ? 8 : 4;
}

int blocks_per_cu(int waves) { return waves == 4 ? 2 : 1; }

// Deal sets of work items to the 8 XCDs (largest first onto the least-loaded
// XCD) and interleave them so that item k of XCD x lands at workgroup index
// 8k + x; shorter XCD lists are padded with NOOP items.
template <typename SetT>
static void order_for_xcds(std::vector<SetT>& sets, std::vector<WorkItem>& out) {
  std::stable_sort(sets.begin(), sets.end(), [](const SetT& a, const SetT& b) { return a.cost > b.cost; });
  std::vector<long long> load(8, 0);
  std::vector<std::vector<WorkItem>> lists(8);
  for (auto& set : sets) {
    const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    load[x] += set.cost;
    lists[x].insert(lists[x].end(), set.items.begin(), set.items.end());
  }
  size_t maxlen = 0;
  for (auto& l : lists) maxlen = std::max(maxlen, l.size());
  for (size_t k = 0; k < maxlen; ++k)
    for (int x = 0; x < 8; ++x) {
      if (k < lists[x].size()) {
        out.push_back(lists[x][k]);
      } else {
        WorkItem w{};
        w.mode = MODE_NOOP;
        out.push_back(w);
      }
    }
  while (!out.empty() && out.back().mode == MODE_NOOP) out.pop_back();
}

int plan_cascade(const PlanInput& in, PlanOutput& out) {
  out.prefix_work.clear();
  out.suffix_work.clear();
  const int Hkv = in.num_kv_heads;
  const int g = in.num_qo_heads / Hkv;
  int max_rows = 0;
  for (int r = 0; r < in.num_reqs; ++r) max_rows = std::max(max_rows, (in.qo_indptr[r + 1] - in.qo_indptr[r]) * g);
  const int WA = in.waves ? in.waves : choose_waves(max_rows);
  const int ROWS_A = 32 * WA;
  const int WB = kSuffixWaves;  // divides WA, so a suffix block lies in one prefix tile
  const int ROWS_B = 32 * WB;
  const int num_cus = in.num_cus > 0 ? in.num_cus : 256;
  const long long target = (long long)num_cus * blocks_per_cu(WA);

  const int R = in.num_reqs;
  std::vector<int> qtiles(R), ptiles(R), kv0(R), kv1(R), splits(R, 0), nq(R);
  long long prefix_cost = 0;
  for (int r = 0; r < R; ++r) {
    nq[r] = in.qo_indptr[r + 1] - in.qo_indptr[r];
    qtiles[r] = (nq[r] * g + ROWS_A - 1) / ROWS_A;
    const int L = in.prefix_len[r];
    const int Leff = in.window_left >= 0 ? std::min(L, in.window_left) : L;
    kv0[r] = L - Leff;
    kv1[r] = L;
    ptiles[r] = nq[r] > 0 ? (Leff + 63) / 64 : 0;
    prefix_cost += (long long)Hkv * qtiles[r] * ptiles[r];
  }
  // Key tiles per prefix split: the smallest chunk for which one wave of
  // workgroups covers the prefix level, capped so that one split's page ids
  // fit the kernel's LDS staging area.
  int chunk = 1;
  if (prefix_cost > 0) {
    chunk = (int)std::max<long long>(1, (prefix_cost + target - 1) / target);
    auto wgs = [&](int c) {
      long long t = 0;
      for (int r = 0; r < R; ++r) t += (long long)Hkv * qtiles[r] * ((ptiles[r] + c - 1) / c);
      return t;
    };
    // once every request is a single split, more chunking cannot help
    int max_ptiles = 1;
    for (int r = 0; r < R; ++r) max_ptiles = std::max(max_ptiles, ptiles[r]);
    while (chunk < max_ptiles && wgs(chunk) > target) ++chunk;
    if (in.page_size > 0) {
      const int max_chunk = std::max(1, ((kMaxStagedPages - 2) * in.page_size) / 64);
      chunk = std::min(chunk, max_chunk);
    }
  }

  // slot_begin per group (r, h, qt): S_r consecutive partial slots.
  std::vector<int> grp0(R + 1, 0);
  for (int r = 0; r < R; ++r) grp0[r + 1] = grp0[r] + Hkv * qtiles[r];
  std::vector<int> slot_begin(grp0[R], -1);
  int slot = 0, max_splits_used = 0;
  for (int r = 0; r < R; ++r) {
    int s = ptiles[r] == 0 ? 0 : (ptiles[r] + chunk - 1) / chunk;
    if (in.max_splits > 0) s = std::min(s, in.max_splits);
    splits[r] = s;
    max_splits_used = std::max(max_splits_used, s);
    for (int gi = grp0[r]; gi < grp0[r + 1]; ++gi) {
      if (s > 0) slot_begin[gi] = slot;
      slot += s;
    }
  }

  // Sets of work items that read the same keys (placed on one XCD).
  struct Set {
    long long cost;
    std::vector<WorkItem> items;
  };
  std::vector<Set> pre_sets, suf_sets;
  for (int r = 0; r < R; ++r) {
    if (nq[r] == 0) continue;
    const int S = splits[r];
    for (int h = 0; h < Hkv; ++h) {
      for (int s = 0; s < S; ++s) {
        const int base = ptiles[r] / S, rem = ptiles[r] % S;
        const int t0 = s * base + std::min(s, rem);
        const int nt = base + (s < rem ? 1 : 0);
        Set set;
        set.cost = (long long)nt * qtiles[r];
        for (int qt = 0; qt < qtiles[r]; ++qt) {
          WorkItem w;
          w.req = r;
          w.kvh = h;
          w.qtile = qt;
          w.src = 0;
          w.kv_begin = kv0[r] + 64 * t0;
          w.kv_end = std::min(kv1[r], kv0[r] + 64 * (t0 + nt));
          w.slot = slot_begin[grp0[r] + h * qtiles[r] + qt] + s;
          w.mode = MODE_PARTIAL;
          set.items.push_back(w);
        }
        pre_sets.push_back(std::move(set));
      }
      const int nb = (nq[r] * g + ROWS_B - 1) / ROWS_B;
      Set set;
      set.cost = (long long)nb * ((nq[r] + 63) / 64);
      for (int b = 0; b < nb; ++b) {
        const int qt = (b * ROWS_B) / ROWS_A;
        WorkItem w;
        w.req = r;
        w.kvh = h;
        w.qtile = b;
        w.src = 1;
        w.kv_begin = 0;
        w.kv_end = nq[r];
        if (S > 0) {
          w.slot = slot_begin[grp0[r] + h * qtiles[r] + qt];
          w.mode = MODE_MERGE_SLOTS | (S << 8);
        } else {
          w.slot = -1;
          w.mode = MODE_FINAL;
        }
        set.items.push_back(w);
      }
      suf_sets.push_back(std::move(set));
    }
  }
  order_for_xcds(pre_sets, out.prefix_work);
  order_for_xcds(suf_sets, out.suffix_work);

  out.waves = WA;
  out.suffix_waves = WB;
  out.rows_per_tile = ROWS_A;
  out.num_slots = slot;
  out.max_splits_used = max_splits_used;
  // bf16 partial O + fp32 LSE per (slot, row)
  out.workspace_bytes = (size_t)slot * ROWS_A * ((size_t)in.head_dim * 2 + sizeof(float));
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
      splits > 1 ? (size_t)groups * splits * ROWS * ((size_t)head_dim * 2 + sizeof(float)) : 0;
}

}  // namespace d2sd
