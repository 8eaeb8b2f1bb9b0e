// Host-side work planning for cascade verify attention (plan()) and the
// single-source drop-in (single_prefill_with_kv_cache).
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
// 8k + x (workgroups are dispatched to XCDs round-robin); shorter XCD lists are
// padded with NOOP items.
template <typename Item>
struct ItemSet {
  long long cost;
  std::vector<Item> items;
};

// Returns, per input set (input order), the XCD it was dealt to.
template <typename Item>
static std::vector<int> order_for_xcds(std::vector<ItemSet<Item>>& sets, std::vector<Item>& out) {
  std::vector<int> idx(sets.size());
  for (size_t i = 0; i < idx.size(); ++i) idx[i] = (int)i;
  std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return sets[a].cost > sets[b].cost; });
  std::vector<long long> load(8, 0);
  std::vector<std::vector<Item>> lists(8);
  std::vector<int> xcd_of(sets.size(), 0);
  for (int i : idx) {
    const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    load[x] += sets[i].cost;
    xcd_of[i] = x;
    lists[x].insert(lists[x].end(), sets[i].items.begin(), sets[i].items.end());
  }
  size_t maxlen = 0;
  for (auto& l : lists) maxlen = std::max(maxlen, l.size());
  for (size_t k = 0; k < maxlen; ++k)
    for (int x = 0; x < 8; ++x) {
      if (k < lists[x].size()) {
        out.push_back(lists[x][k]);
      } else {
        Item w{};
        w.mode = MODE_NOOP;
        out.push_back(w);
      }
    }
  while (!out.empty() && out.back().mode == MODE_NOOP) out.pop_back();
  return xcd_of;
}

// Interleave per-XCD merge lists: merge workgroup 8k + x runs on XCD x.
static void interleave_merges(const std::vector<std::vector<VerifyMerge>>& lists, std::vector<VerifyMerge>& out) {
  size_t maxlen = 0;
  for (auto& l : lists) maxlen = std::max(maxlen, l.size());
  for (size_t k = 0; k < maxlen; ++k)
    for (int x = 0; x < 8; ++x) {
      if (k < lists[x].size()) {
        out.push_back(lists[x][k]);
      } else {
        VerifyMerge m{};
        m.nslots = 0;  // padding: no work
        out.push_back(m);
      }
    }
  while (!out.empty() && out.back().nslots == 0) out.pop_back();
}

int verify_wgs_per_cu(int waves) { return waves == 8 ? 1 : 2; }
int verify_rows(int waves) { return waves == 2 ? 128 : 32 * waves; }

// Waves per workgroup when the caller leaves it to the planner: 4 (128-row
// q-tiles, two workgroups per CU) by default; 8 (256-row q-tiles, one per CU)
// when the 4-wave plan already has at least one q-tile group per workgroup
// slot, so that the prefix would not be split anyway, and some kv head packs
// more than 128 rows: each K/V tile staged in LDS then feeds twice the rows
// (measured: Qwen3-32B shape, 32 requests x 8192 keys, 4565 queries: 1790
// vs 2125 us per attention launch).  Where the prefix must be split to fill
// the device the finer 4-wave tiles balance better.
int verify_auto_waves(const VerifyPlanInput& in, int num_cus) {
  const int Hkv = in.num_kv_heads;
  const int g = in.num_qo_heads / Hkv;
  long long groups = 0;
  int max_rows = 0;
  for (int r = 0; r < in.num_reqs; ++r) {
    const int nq = in.qo_indptr[r + 1] - in.qo_indptr[r];
    if (nq <= 0 || in.prefix_len[r] <= 0) continue;
    max_rows = std::max(max_rows, nq * g);
    groups += (long long)Hkv * ((nq * g + verify_rows(4) - 1) / verify_rows(4));
  }
  return max_rows > verify_rows(4) && groups >= (long long)num_cus * verify_wgs_per_cu(4) ? 8 : 4;
}

// Cascade verify plan.  Groups are (request, kv head, q-tile of ROWS packed
// rows).  Each group gets S key chunks of its visible prefix (S partial
// slots) plus one suffix item (slot S), merged by one merge item; a group
// with no prefix keys has only its suffix item, which writes the output.
// The chunk length is the smallest that keeps every item of the launch
// resident at once (verify_wgs_per_cu per CU), capped so that S stays within
// kMaxVerifySplits and a chunk's page ids fit the kernel's LDS staging.
int plan_verify(const VerifyPlanInput& in, VerifyPlanOutput& out) {
  out.items.clear();
  out.merges.clear();
  const int Hkv = in.num_kv_heads;
  const int g = in.num_qo_heads / Hkv;
  const int R = in.num_reqs;
  const int num_cus = in.num_cus > 0 ? in.num_cus : 256;
  const int W = in.waves ? in.waves : verify_auto_waves(in, num_cus);
  const int ROWS = verify_rows(W);
  const long long capacity = (long long)num_cus * verify_wgs_per_cu(W);
  const int split_cap =
      in.max_splits > 0 ? std::min(in.max_splits, kMaxVerifySplits) : kMaxVerifySplits;

  std::vector<int> nq(R), qtiles(R), ptiles(R), stiles(R), kv0(R), kv1(R), splits(R, 0);
  long long units = 0, groups = 0;
  int max_ptiles = 1;
  for (int r = 0; r < R; ++r) {
    nq[r] = in.qo_indptr[r + 1] - in.qo_indptr[r];
    qtiles[r] = (nq[r] * g + ROWS - 1) / ROWS;
    const int L = in.prefix_len[r];
    const int Leff = in.window_left >= 0 ? std::min(L, in.window_left) : L;
    kv0[r] = L - Leff;
    kv1[r] = L;
    ptiles[r] = nq[r] > 0 ? (Leff + 63) / 64 : 0;
    stiles[r] = (nq[r] + 63) / 64;
    max_ptiles = std::max(max_ptiles, ptiles[r]);
    units += (long long)Hkv * qtiles[r] * (ptiles[r] + stiles[r]);
    groups += (long long)Hkv * qtiles[r];
  }
  auto wgs = [&](int c) {
    long long t = 0;
    for (int r = 0; r < R; ++r)
      if (nq[r] > 0) t += (long long)Hkv * qtiles[r] * ((ptiles[r] + c - 1) / c + 1);
    return t;
  };
  int chunk = (int)std::max<long long>(1, (units + capacity - 1) / std::max<long long>(capacity, 1));
  while (chunk < max_ptiles && wgs(chunk) > capacity) ++chunk;
  for (int r = 0; r < R; ++r) chunk = std::max(chunk, (ptiles[r] + split_cap - 1) / split_cap);
  if (in.page_size > 0) {
    const int max_chunk = std::max(1, ((kMaxStagedPages - 8) * in.page_size) / 64);
    chunk = std::min(chunk, max_chunk);
  }
  (void)groups;

  // consecutive slots per group: S prefix partials, then the suffix partial
  std::vector<int> grp0(R + 1, 0);
  for (int r = 0; r < R; ++r) grp0[r + 1] = grp0[r] + Hkv * qtiles[r];
  std::vector<int> slot0(grp0[R], -1);
  int slot = 0, max_splits_used = 0;
  for (int r = 0; r < R; ++r) {
    const int S = ptiles[r] == 0 ? 0 : (ptiles[r] + chunk - 1) / chunk;
    splits[r] = S;
    max_splits_used = std::max(max_splits_used, S);
    for (int gi = grp0[r]; gi < grp0[r + 1]; ++gi) {
      if (S > 0) {
        slot0[gi] = slot;
        slot += S + 1;
      }
    }
  }

  // One set per (request, kv head): all its q-tiles, key chunks and suffix
  // items run on one XCD, so the head's K/V and Q come from HBM once and its
  // partial states stay in that XCD's L2.  With fewer such sets than XCDs,
  // each key chunk (with all q-tiles reading it) is a set of its own.
  long long nheads_sets = 0;
  for (int r = 0; r < R; ++r) nheads_sets += nq[r] > 0 ? Hkv : 0;
  const bool per_head = nheads_sets >= 8;
  std::vector<ItemSet<VerifyItem>> sets;
  std::vector<std::vector<VerifyMerge>> set_merges;
  for (int r = 0; r < R; ++r) {
    if (nq[r] == 0) continue;
    const int S = splits[r];
    const int q0 = in.qo_indptr[r];
    const int pbase = in.page_size > 0 ? in.page_indptr[r] : (in.prefix_tok_indptr ? in.prefix_tok_indptr[r] : 0);
    for (int h = 0; h < Hkv; ++h) {
      ItemSet<VerifyItem> head_set;
      head_set.cost = 0;
      for (int s_ = 0; s_ < S; ++s_) {
        const int base = ptiles[r] / S, rem = ptiles[r] % S;
        const int t0 = s_ * base + std::min(s_, rem);
        const int nt = base + (s_ < rem ? 1 : 0);
        ItemSet<VerifyItem> set;
        set.cost = (long long)nt * qtiles[r];
        for (int qt = 0; qt < qtiles[r]; ++qt) {
          VerifyItem w{};
          w.req = r;
          w.kvh = h;
          w.qtile = qt;
          w.src = SRC_PREFIX;
          w.kv_begin = kv0[r] + 64 * t0;
          w.kv_end = std::min(kv1[r], kv0[r] + 64 * (t0 + nt));
          w.slot = slot0[grp0[r] + h * qtiles[r] + qt] + s_;
          w.mode = MODE_PARTIAL;
          w.group = grp0[r] + h * qtiles[r] + qt;
          w.slot0 = slot0[w.group];
          w.nprod = S + 1;
          w.q0 = q0;
          w.nq = nq[r];
          w.base = pbase;
          w.causal_off = 0;
          set.items.push_back(w);
        }
        if (per_head) {
          head_set.cost += set.cost;
          head_set.items.insert(head_set.items.end(), set.items.begin(), set.items.end());
        } else {
          sets.push_back(std::move(set));
          set_merges.emplace_back();
        }
      }
      ItemSet<VerifyItem> set;
      set.cost = (long long)stiles[r] * qtiles[r];
      std::vector<VerifyMerge> merges;
      for (int qt = 0; qt < qtiles[r]; ++qt) {
        const int gi = grp0[r] + h * qtiles[r] + qt;
        VerifyItem w{};
        w.req = r;
        w.kvh = h;
        w.qtile = qt;
        w.src = SRC_SUFFIX;
        w.kv_begin = 0;
        w.kv_end = nq[r];
        w.slot = S > 0 ? slot0[gi] + S : -1;
        w.mode = S > 0 ? MODE_PARTIAL : MODE_FINAL;
        w.group = gi;
        w.slot0 = S > 0 ? slot0[gi] : -1;
        w.nprod = S + 1;
        w.q0 = q0;
        w.nq = nq[r];
        w.base = q0;  // the request's suffix keys are rows q0.. of k/v_suffix
        w.causal_off = 0;
        set.items.push_back(w);
        if (S > 0) {
          // one merge workgroup per 32-row block holding valid rows
          for (int blk = 0; blk < ROWS / 32 && qt * ROWS + blk * 32 < nq[r] * g; ++blk) {
            VerifyMerge m{};
            m.req = r;
            m.kvh = h;
            m.qtile = qt;
            m.slot0 = slot0[gi];
            m.nslots = S + 1;
            m.q0 = q0;
            m.nq = nq[r];
            m.blk = blk;
            merges.push_back(m);
          }
        }
      }
      if (per_head) {
        head_set.cost += set.cost;
        head_set.items.insert(head_set.items.end(), set.items.begin(), set.items.end());
        sets.push_back(std::move(head_set));
        set_merges.push_back(std::move(merges));
      } else {
        sets.push_back(std::move(set));
        set_merges.push_back(std::move(merges));
      }
    }
  }
  const std::vector<int> xcd = order_for_xcds(sets, out.items);
  std::vector<std::vector<VerifyMerge>> mlists(8);
  for (size_t i = 0; i < set_merges.size(); ++i)
    mlists[xcd[i]].insert(mlists[xcd[i]].end(), set_merges[i].begin(), set_merges[i].end());
  interleave_merges(mlists, out.merges);

  out.waves = W;
  out.rows = ROWS;
  out.num_slots = slot;
  out.max_splits_used = max_splits_used;
  out.num_groups = grp0[R];
  out.merge_mode = slot > 0 ? in.merge_mode : MERGE_LAUNCH;
  out.merge_in_attention = out.merge_mode != MERGE_LAUNCH;
  if (out.merge_in_attention) out.merges.clear();
  // bf16 partial O + fp32 LSE per (slot, row), then the int32 counters
  // (16-byte aligned)
  const size_t part_bytes = (size_t)slot * ROWS * ((size_t)in.head_dim * 2 + sizeof(float));
  out.counters_offset = (part_bytes + 15) & ~(size_t)15;
  out.workspace_bytes = out.merge_in_attention ? out.counters_offset + (size_t)out.num_groups * sizeof(int)
                                               : part_bytes;
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
