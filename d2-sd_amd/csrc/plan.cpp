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

// Cascade verify plan.
//
// Groups are (request, kv head, q-tile of ROWS packed rows); each group's
// visible prefix is cut into key chunks (split-KV), one partial state each,
// plus one suffix (tree) item, and the merge launch combines the group's
// partials.  A group with no prefix keys has only its suffix item, which
// writes the output.
//
// Placement.  Workgroups are dealt to the 8 XCDs round-robin (workgroup i on
// XCD i % 8), and inside an XCD the k-th workgroup of the first round and the
// k-th of the second round land on the same CU (measured on MI355X with
// per-workgroup HW_ID / XCC_ID reads).  Sets = all q-tiles of one (request,
// kv head), or of one key range of it when there are fewer than 8 such sets,
// so that every key tile is read from HBM once and re-read from that XCD's
// L2 by the other q-tiles; sets go to XCDs largest first onto the least-loaded
// XCD.
//
// Balance.  Per XCD the prefix chunks are sized to fill its workgroup slots
// (CUs per XCD x workgroups per CU) after the suffix items: the largest chunk
// T is the smallest that fits, then the remaining slots split the groups whose
// chunks are longest.  Where those chunks are at least 4 tiles long and one
// workgroup per CU (the suffix items paired with each other) needs chunks
// less than 1.6x as long, the chunks are sized for that instead: a lone
// workgroup steps through tiles faster than two that share a CU.  With one or two rounds of workgroups per XCD, the
// longest items run alone and the rest are paired longest-with-shortest on a
// CU; beyond two rounds items go longest first.
namespace {

struct Piece {            // the q-tiles of one (request, kv head) over prefix tiles [t0, t1)
  int req, kvh, t0, t1;
  bool suffix;            // the set's q-tiles also get their suffix items here
};

struct PlanItem {
  VerifyItem w;
  int cost;               // in prefix-tile units
  int c = -1;             // a whole-prefix chunk's index among its group's chunks (else -1)
};

int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

}  // namespace

int plan_verify(const VerifyPlanInput& in, VerifyPlanOutput& out) {
  out.items.clear();
  out.merges.clear();
  const int Hkv = in.num_kv_heads;
  const int g = in.num_qo_heads / Hkv;
  const int R = in.num_reqs;
  const int num_cus = in.num_cus > 0 ? in.num_cus : 256;
  const int W = in.waves ? in.waves : verify_auto_waves(in, num_cus);
  const int ROWS = verify_rows(W);
  const int wpc = verify_wgs_per_cu(W);
  const int cus_per_xcd = std::max(1, num_cus / 8);
  const int xcd_slots = cus_per_xcd * wpc;
  const int split_cap = in.max_splits > 0 ? std::min(in.max_splits, kMaxVerifySplits) : kMaxVerifySplits;
  // A chunk's page ids must fit the kernel's LDS staging; this bound wins over
  // split_cap (a group then has more than split_cap chunks, which the merge
  // takes in batches).
  const int max_chunk = verify_max_chunk_tiles(in.page_size);
  constexpr int kMinChunk = 2;  // shorter chunks cost more in partials than they gain in balance

  // A two-segment prefix (in.prefix_split) is tiled segment by segment: the
  // first segment's tiles start at the window start kv0 (its last tile ends
  // at the split, possibly partial), the second's at its own first visible
  // key, so no tile holds keys of both segments.  Tile boundaries of request
  // r: key kv0 + 64 t for t <= ta[r], then second-segment key b0[r] + 64 (t - ta[r]).
  std::vector<int> nq(R), qtiles(R), ptiles(R), stiles(R), kv0(R), kv1(R), sp(R), ta(R), b0(R);
  bool second = false;  // some request sees keys of the second segment
  for (int r = 0; r < R; ++r) {
    nq[r] = in.qo_indptr[r + 1] - in.qo_indptr[r];
    qtiles[r] = (nq[r] * g + ROWS - 1) / ROWS;
    const int L = in.prefix_len[r];
    const int Leff = in.window_left >= 0 ? std::min(L, in.window_left) : L;
    kv0[r] = L - Leff;
    kv1[r] = L;
    sp[r] = in.prefix_split ? std::min(std::max(in.prefix_split[r], 0), L) : L;
    ta[r] = sp[r] > kv0[r] ? (sp[r] - kv0[r] + 63) / 64 : 0;
    b0[r] = std::max(kv0[r], sp[r]) - sp[r];
    const int tb = (L - sp[r] - b0[r] + 63) / 64;
    ptiles[r] = nq[r] > 0 ? ta[r] + tb : 0;
    second = second || (nq[r] > 0 && tb > 0);
    stiles[r] = (nq[r] + 63) / 64;
  }
  std::vector<int> grp0(R + 1, 0);
  for (int r = 0; r < R; ++r) grp0[r + 1] = grp0[r] + Hkv * qtiles[r];
  const int ngroups = grp0[R];

  // ---- sets of pieces, dealt to XCDs ----
  int nsets = 0;
  for (int r = 0; r < R; ++r) nsets += nq[r] > 0 ? Hkv : 0;
  std::vector<std::vector<Piece>> sets;
  std::vector<long long> set_cost;
  for (int r = 0; r < R; ++r) {
    if (nq[r] == 0) continue;
    const int ranges = (nsets >= 8 || ptiles[r] == 0) ? 1
                       : std::min({ceil_div(8, nsets), ptiles[r], split_cap});
    for (int h = 0; h < Hkv; ++h)
      for (int k = 0; k < ranges; ++k) {
        Piece pc{r, h, (int)((long long)ptiles[r] * k / ranges), (int)((long long)ptiles[r] * (k + 1) / ranges),
                 k == 0};
        sets.push_back({pc});
        set_cost.push_back((long long)qtiles[r] * ((pc.t1 - pc.t0) + (pc.suffix ? 2 * stiles[r] : 0)));
      }
  }
  std::vector<int> order(sets.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return set_cost[a] > set_cost[b]; });
  std::vector<long long> load(8, 0);
  std::vector<std::vector<int>> xcd_sets(8);
  for (int s : order) {
    const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    load[x] += set_cost[s];
    xcd_sets[x].push_back(s);
  }

  // ---- chunk counts per (piece, q-tile), XCD by XCD ----
  // nchunk[set][qt]: prefix chunks of q-tile qt of the set's piece
  std::vector<std::vector<int>> nchunk(sets.size());
  for (int x = 0; x < 8; ++x) {
    struct Cell { int set, qt, pt, cap; };
    std::vector<Cell> cells;
    int suffix_items = 0;
    for (int s : xcd_sets[x]) {
      const Piece& pc = sets[s][0];
      nchunk[s].assign(qtiles[pc.req], 0);
      const int pieces_per_group = (nsets >= 8 || ptiles[pc.req] == 0) ? 1
                                   : std::min({ceil_div(8, nsets), ptiles[pc.req], split_cap});
      const int cap = std::max(1, split_cap / pieces_per_group);
      for (int qt = 0; qt < qtiles[pc.req]; ++qt) {
        if (pc.t1 > pc.t0) cells.push_back({s, qt, pc.t1 - pc.t0, cap});
        if (pc.suffix) ++suffix_items;
      }
    }
    if (cells.empty()) continue;
    int maxpt = 1, tmin = 1;
    for (auto& c : cells) {
      maxpt = std::max(maxpt, c.pt);
      tmin = std::max(tmin, ceil_div(c.pt, c.cap));
    }
    auto count = [&](int t) {
      long long n = 0;
      for (auto& c : cells) n += ceil_div(c.pt, t);
      return n;
    };
    // the longest chunk that fits `slots` items
    auto chunk_len = [&](long long slots) {
      int t = std::max(tmin, std::min(kMinChunk, maxpt));
      while (t < maxpt && count(t) > slots) ++t;
      return t;
    };
    long long budget = std::max<long long>((long long)xcd_slots - suffix_items, (long long)cells.size());
    int T = chunk_len(budget);
    if (wpc == 2 && T >= 4) {
      // One workgroup per CU (the suffix items paired with each other)
      // instead of two: a lone workgroup steps through a tile in about 1.45
      // us, each of two sharing a CU in 1.8-2.0 us, so the lone plan's
      // longer chunks can end first.  Measured on MI355X, 96 nodes, 24
      // q-tile groups: 4096 keys, 7 tiles alone 12.3 us per attention launch
      // against 4-5 paired 13.2 us (1.4x the length); 8192 keys, 13 alone
      // 20.6 us against 9 paired 22.0 us (1.44x); at 2x and 2.2x (128 and
      // 150 nodes) the lone plan lost, so the bound is 1.6x.  Below 4 tiles
      // per paired chunk the per-item fixed cost, which two workgroups of a
      // CU overlap, dominates (2048 keys: 3 paired 14.5 us per call against
      // 4 alone 14.9 us).
      const long long alone = std::max<long long>((long long)cus_per_xcd - (suffix_items + 1) / 2,
                                                  (long long)cells.size());
      const int Ta = chunk_len(alone);
      if (5 * Ta < 8 * T) {
        budget = alone;
        T = Ta;
      }
    }
    T = std::min(T, max_chunk);
    long long used = 0;
    std::vector<int> n(cells.size());
    for (size_t i = 0; i < cells.size(); ++i) {
      n[i] = ceil_div(cells[i].pt, T);
      used += n[i];
    }
    // remaining slots: one more chunk to the cell whose chunks are longest
    // (most chunks at that length first), while chunks stay >= kMinChunk
    for (long long extra = budget - used; extra > 0; --extra) {
      int best = -1;
      long long best_key = -1;
      for (size_t i = 0; i < cells.size(); ++i) {
        const int len = ceil_div(cells[i].pt, n[i]);
        if (n[i] + 1 > cells[i].cap || cells[i].pt / (n[i] + 1) < kMinChunk) continue;
        const int at_len = cells[i].pt % n[i] ? cells[i].pt % n[i] : n[i];
        const long long key = (long long)len * 4096 + at_len;
        if (key > best_key) { best_key = key; best = (int)i; }
      }
      if (best < 0) break;
      ++n[best];
    }
    for (size_t i = 0; i < cells.size(); ++i) nchunk[cells[i].set][cells[i].qt] = n[i];
  }

  // ---- partial slots: per group its prefix chunks in key order, then the suffix ----
  // Chunk c of S over tiles [t0, t1): tiles [t0 + span c / S, t0 + span (c+1) / S);
  // a chunk of a request's whole visible prefix takes the partition
  // dyn_chunk_start (the first span % S chunks one tile longer), which a
  // dynamic plan's kernels repeat at the run-time length.  A chunk holding
  // tiles of both segments is cut at the split: two items.
  auto whole = [&](const Piece& pc) { return !in.prefix_split && pc.t0 == 0 && pc.t1 == ptiles[pc.req]; };
  auto chunk_tiles = [&](const Piece& pc, int S, int c, int& a, int& b) {
    const int span = pc.t1 - pc.t0;
    if (whole(pc)) {
      a = pc.t0 + dyn_chunk_start(c, S, span);
      b = pc.t0 + dyn_chunk_start(c + 1, S, span);
      return;
    }
    a = pc.t0 + (int)((long long)span * c / S);
    b = pc.t0 + (int)((long long)span * (c + 1) / S);
  };
  std::vector<int> gchunks(ngroups, 0);
  for (size_t s = 0; s < sets.size(); ++s) {
    const Piece& pc = sets[s][0];
    for (int qt = 0; qt < qtiles[pc.req]; ++qt) {
      int& gc = gchunks[grp0[pc.req] + pc.kvh * qtiles[pc.req] + qt];
      gc += nchunk[s][qt];
      for (int c = 0; c < nchunk[s][qt]; ++c) {
        int a, b;
        chunk_tiles(pc, nchunk[s][qt], c, a, b);
        gc += a < ta[pc.req] && ta[pc.req] < b;
      }
    }
  }
  // When no group's prefix is split, one item per group reads the group's
  // prefix and then its suffix tree (SRC_BOTH) and writes the output: the
  // plan has no partial states and no merge launch.  Plans that read a
  // second prefix segment are never fused.
  bool fuse = !second;
  for (int gi = 0; gi < ngroups; ++gi) fuse = fuse && gchunks[gi] <= 1;
  std::vector<int> slot0(ngroups, -1), next_slot(ngroups, 0);
  int slot = 0, max_splits_used = 0;
  for (int gi = 0; gi < ngroups; ++gi) {
    max_splits_used = std::max(max_splits_used, gchunks[gi]);
    if (gchunks[gi] > 0 && !fuse) {
      slot0[gi] = slot;
      next_slot[gi] = slot;
      slot += gchunks[gi] + 1;
    }
  }

  // ---- items per XCD (sets in key order within a group, so slots follow key order) ----
  std::vector<std::vector<PlanItem>> lists(8);
  std::vector<std::vector<VerifyMerge>> mlists(8);
  std::vector<int> set_order(sets.size());
  for (size_t i = 0; i < set_order.size(); ++i) set_order[i] = (int)i;  // creation order = (req, head, range)
  std::vector<int> set_xcd(sets.size(), 0);
  for (int x = 0; x < 8; ++x)
    for (int s : xcd_sets[x]) set_xcd[s] = x;
  for (int s : set_order) {
    const Piece& pc = sets[s][0];
    const int r = pc.req, h = pc.kvh, x = set_xcd[s];
    const int q0 = in.qo_indptr[r];
    const int pbase = in.page_size > 0 ? in.page_indptr[r] : (in.prefix_tok_indptr ? in.prefix_tok_indptr[r] : 0);
    const int pbase2 = in.prefix2_tok_indptr ? in.prefix2_tok_indptr[r] : 0;
    for (int qt = 0; qt < qtiles[r]; ++qt) {
      const int gi = grp0[r] + h * qtiles[r] + qt;
      const int S = nchunk[s][qt];
      for (int c = 0; c < S; ++c) {
        int a, b;
        chunk_tiles(pc, S, c, a, b);
        VerifyItem w{};
        w.req = r;
        w.kvh = h;
        w.qtile = qt;
        w.mode = fuse ? MODE_FINAL : MODE_PARTIAL;
        w.q0 = q0;
        w.nq = nq[r];
        if (a < ta[r]) {  // first segment: keys [kv0 + 64 a, min(kv0 + 64 b, split))
          const int e = std::min(b, ta[r]);
          w.src = fuse ? SRC_BOTH : SRC_PREFIX;
          w.kv0 = kv0[r];
          w.plan_len = kv1[r];
          w.kv_begin = kv0[r] + 64 * a;
          w.kv_end = std::min(sp[r], kv0[r] + 64 * e);
          w.slot = fuse ? -1 : next_slot[gi]++;
          w.base = pbase;
          // a chunk of the whole visible prefix names its place in the
          // partition (dynamic plans repeat it on the device); a dynamic
          // plan's pieces of a range scale their planned boundaries instead
          const bool wh = whole(pc);
          w.chunk = wh ? c | S << 16 : 0;
          lists[x].push_back({w, (e - a) + (fuse ? 2 * stiles[r] : 0), wh ? c : -1});
        }
        if (b > ta[r]) {  // second segment, in its own key numbering
          const int f = std::max(a, ta[r]);
          const int len2 = kv1[r] - sp[r];
          w.src = SRC_PREFIX2;
          w.kv0 = b0[r];
          w.plan_len = len2;
          w.kv_begin = b0[r] + 64 * (f - ta[r]);
          w.kv_end = std::min(len2, b0[r] + 64 * (b - ta[r]));
          w.slot = next_slot[gi]++;
          w.base = pbase2;
          lists[x].push_back({w, b - f});
        }
      }
    }
    if (!pc.suffix) continue;
    for (int qt = 0; qt < qtiles[r]; ++qt) {
      const int gi = grp0[r] + h * qtiles[r] + qt;
      if (fuse && gchunks[gi] == 1) continue;  // its SRC_BOTH item reads the suffix
      const bool split = gchunks[gi] > 0;
      VerifyItem w{};
      w.req = r;
      w.kvh = h;
      w.qtile = qt;
      w.src = SRC_SUFFIX;
      w.kv_begin = 0;
      w.kv_end = nq[r];
      w.slot = split ? slot0[gi] + gchunks[gi] : -1;
      w.mode = split ? MODE_PARTIAL : MODE_FINAL;
      w.q0 = q0;
      w.nq = nq[r];
      w.base = q0;  // the request's suffix keys are rows q0.. of k/v_suffix
      lists[x].push_back({w, 2 * stiles[r]});
      if (split)  // one merge workgroup per 32-row block holding valid rows
        for (int blk = 0; blk < ROWS / 32 && qt * ROWS + blk * 32 < nq[r] * g; ++blk) {
          VerifyMerge m{};
          m.req = r;
          m.kvh = h;
          m.qtile = qt;
          m.slot0 = slot0[gi];
          m.nslots = gchunks[gi] + 1;
          m.q0 = q0;
          m.nq = nq[r];
          m.blk = blk;
          mlists[x].push_back(m);
        }
    }
  }

  // ---- dispatch order per XCD, then interleave the XCDs ----
  std::vector<std::vector<VerifyItem>> ordered(8);
  for (int x = 0; x < 8; ++x) {
    auto& L = lists[x];
    // longest first, ties to lower chunk indices first: a group's first
    // chunks (the ones the partition lengthens first) run in the first round,
    // each paired with a later chunk
    std::stable_sort(L.begin(), L.end(), [](const PlanItem& a, const PlanItem& b) {
      return a.cost != b.cost ? a.cost > b.cost : a.c < b.c;
    });
    const int m = (int)L.size(), K = cus_per_xcd;
    auto& o = ordered[x];
    if (wpc == 2 && m > K && m <= 2 * K) {
      // p CUs run a pair, K - p run one item: first round = the pairs' longer
      // halves, then the singles (the longest items); second round = the
      // pairs' shorter halves, k-th with k-th
      const int p = m - K, s = K - p;
      for (int i = 0; i < p; ++i) o.push_back(L[s + i].w);
      for (int i = 0; i < s; ++i) o.push_back(L[i].w);
      for (int i = 0; i < p; ++i) o.push_back(L[m - 1 - i].w);
    } else {
      for (auto& it : L) o.push_back(it.w);
    }
  }
  size_t maxlen = 0;
  for (auto& l : ordered) maxlen = std::max(maxlen, l.size());
  for (size_t k = 0; k < maxlen; ++k)
    for (int x = 0; x < 8; ++x) {
      if (k < ordered[x].size()) {
        out.items.push_back(ordered[x][k]);
      } else {
        VerifyItem w{};
        w.mode = MODE_NOOP;
        out.items.push_back(w);
      }
    }
  while (!out.items.empty() && out.items.back().mode == MODE_NOOP) out.items.pop_back();
  interleave_merges(mlists, out.merges);

  out.waves = W;
  out.rows = ROWS;
  out.num_slots = slot;
  out.max_splits_used = max_splits_used;
  out.num_groups = ngroups;
  out.fused = fuse && max_splits_used > 0 ? 1 : 0;
  // bf16 partial O + fp32 LSE per (slot, row)
  out.workspace_bytes = (size_t)slot * ROWS * ((size_t)in.head_dim * 2 + sizeof(float));
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
