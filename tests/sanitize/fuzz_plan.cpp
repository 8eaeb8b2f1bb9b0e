// Randomized inputs to the cascade planner (d2-sd_amd/csrc/plan.cpp), built
// with AddressSanitizer and UBSan on the host by tests/test_plan_sanitize.py:
// every emitted item reads keys inside its request and segment, paged chunks
// stay within the staged page bound, partial slots are unique and every merge
// names slots that each one item of its group writes, every group's suffix
// tree is read once; the chunks of a group's whole prefix are numbered
// 0..S-1 and their partition (dyn_chunk_start) gives the planned chunks at the
// planned length and tiles every shorter prefix exactly (a dynamic plan's
// run-time chunks), within the staged page bound.
#include <cstdio>
#include <cstdlib>
#include <map>
#include <random>
#include <set>
#include <vector>
#include "plan.h"
using namespace d2sd;
int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 20000;
  std::mt19937_64 rng(12345);
  auto U = [&](int a, int b) { return (int)std::uniform_int_distribution<int>(a, b)(rng); };
  long long checked = 0;
  int fused_plans = 0;
  for (int t = 0; t < iters; ++t) {
    const int R = U(1, 40);
    std::vector<int> qo(R + 1, 0), pl(R), pi(R + 1, 0), ti(R), sp(R), t2(R);
    const int page = std::vector<int>{0, 0, 1, 2, 4, 8, 16, 32, 64}[U(0, 8)];
    const bool two = page == 0 && U(0, 3) == 0;
    for (int r = 0; r < R; ++r) {
      qo[r + 1] = qo[r] + (U(0, 9) == 0 ? 0 : U(1, 300));
      pl[r] = U(0, 9) == 0 ? 0 : U(0, U(0, 1) ? 5000 : 300000 / std::max(1, R));
      if (page) pi[r + 1] = pi[r] + (pl[r] + page - 1) / page + U(0, 2);
      ti[r] = U(0, 1000);
      sp[r] = U(0, pl[r]);
      t2[r] = U(0, 1000);
    }
    const int hkv = std::vector<int>{1, 2, 4, 8}[U(0, 3)];
    const int g = std::vector<int>{1, 2, 4, 8}[U(0, 3)];
    VerifyPlanInput in{};
    in.num_reqs = R;
    in.qo_indptr = qo.data();
    in.prefix_len = pl.data();
    in.page_indptr = page ? pi.data() : nullptr;
    in.prefix_tok_indptr = page ? nullptr : ti.data();
    in.num_qo_heads = hkv * g;
    in.num_kv_heads = hkv;
    in.head_dim = U(0, 1) ? 128 : 64;
    in.window_left = U(0, 3) == 0 ? U(0, 3000) : -1;
    in.num_cus = std::vector<int>{0, 8, 64, 256, 304}[U(0, 4)];
    in.max_splits = U(0, 2) == 0 ? U(1, 20) : 0;
    in.waves = std::vector<int>{0, 2, 4, 8}[U(0, 3)];
    in.page_size = page;
    in.prefix_split = two ? sp.data() : nullptr;
    in.prefix2_tok_indptr = two && U(0, 1) ? t2.data() : nullptr;
    VerifyPlanOutput out{};
    plan_verify(in, out);
    fused_plans += out.fused;
    std::set<int> slots;
    int lg = 0;
    while (page && (1 << lg) < page) ++lg;
    std::map<long long, std::set<int>> chunks;  // group -> chunk indices
    std::map<long long, int> nchunks;
    std::map<long long, int> suffix_readers;    // group -> items reading its suffix tree
    std::map<int, long long> slot_group;        // partial slot -> its writer's group
    for (const auto& w : out.items) {
      if (w.mode == MODE_NOOP) continue;
      ++checked;
      if (w.chunk) {
        const int c = w.chunk & 0xffff, S = w.chunk >> 16;
        const long long key = ((long long)w.req * hkv + w.kvh) * 100000 + w.qtile;
        if ((w.src != SRC_PREFIX && w.src != SRC_BOTH) || c >= S || !chunks[key].insert(c).second ||
            (nchunks.count(key) && nchunks[key] != S)) { printf("bad chunk index\n"); return 1; }
        nchunks[key] = S;
        // the run-time partition of every length up to the planned one
        for (int k = 0; k < 6; ++k) {
          const int L = k == 0 ? pl[w.req] : k == 1 ? 0 : U(0, pl[w.req]);
          const int span = in.window_left >= 0 ? std::min(L, in.window_left) : L, k0 = L - span;
          const int nt = (span + 63) / 64;
          const int b = k0 + std::min(span, 64 * dyn_chunk_start(c, S, nt));
          const int e = k0 + std::min(span, 64 * dyn_chunk_start(c + 1, S, nt));
          const int b0 = k0 + std::min(span, 64 * dyn_chunk_start(0, S, nt));
          const int eS = k0 + std::min(span, 64 * dyn_chunk_start(S, S, nt));
          const int t = (e - b + 63) / 64;
          if (b0 != k0 || eS != L || e < b || t > nt / S + 1 || (nt % S == 0 && t != nt / S) ||
              (k == 0 && (b != w.kv_begin || e != w.kv_end)) ||  // the planned chunk at the planned length
              (page && pages_spanned(b, e, lg) > kMaxStagedPages)) {
            printf("bad run-time chunk L=%d c=%d S=%d [%d, %d)\n", L, c, S, b, e); return 1;
          }
          if (c + 1 < S) {  // contiguous with the next chunk
            const int nb = k0 + std::min(span, 64 * dyn_chunk_start(c + 1, S, nt));
            if (nb != e) { printf("gap\n"); return 1; }
          }
        }
      }
      if (w.req < 0 || w.req >= R || w.kvh < 0 || w.kvh >= hkv) { printf("bad req/kvh\n"); return 1; }
      if (w.src == SRC_SUFFIX) {
        if (w.kv_begin != 0 || w.kv_end != qo[w.req + 1] - qo[w.req]) { printf("bad suffix range\n"); return 1; }
      } else if (w.src == SRC_PREFIX2) {
        if (w.kv_begin < 0 || w.kv_end > pl[w.req] - sp[w.req] || w.kv_begin >= w.kv_end) { printf("bad seg2 range\n"); return 1; }
      } else {
        const int hi = two ? sp[w.req] : pl[w.req];
        if (w.kv_begin < 0 || w.kv_end > hi || w.kv_begin >= w.kv_end) { printf("bad prefix range %d %d %d\n", w.kv_begin, w.kv_end, hi); return 1; }
        if (page && pages_spanned(w.kv_begin, w.kv_end, lg) > kMaxStagedPages) { printf("page bound\n"); return 1; }
      }
      const long long gkey = ((long long)w.req * hkv + w.kvh) * 100000 + w.qtile;
      if (w.src == SRC_SUFFIX || w.src == SRC_BOTH) ++suffix_readers[gkey];
      if (w.src == SRC_BOTH && !out.fused) { printf("SRC_BOTH in a split plan\n"); return 1; }
      if (w.mode == MODE_PARTIAL) {
        if (w.slot < 0 || w.slot >= out.num_slots || !slots.insert(w.slot).second) { printf("bad slot\n"); return 1; }
        slot_group[w.slot] = gkey;
      }
    }
    for (const auto& m : out.merges) {
      if (m.nslots && (m.slot0 < 0 || m.slot0 + m.nslots > out.num_slots)) { printf("bad merge\n"); return 1; }
      const long long gkey = ((long long)m.req * hkv + m.kvh) * 100000 + m.qtile;
      for (int k = 0; k < m.nslots; ++k)  // every merged slot is written by one item of the group
        if (!slot_group.count(m.slot0 + k) || slot_group[m.slot0 + k] != gkey) { printf("unwritten slot\n"); return 1; }
    }
    if ((int)slots.size() != out.num_slots) { printf("slot count\n"); return 1; }
    for (int r = 0; r < R; ++r) {  // every group's suffix tree is read exactly once
      const int n = qo[r + 1] - qo[r];
      if (n == 0) continue;
      const int qt = (n * g + out.rows - 1) / out.rows;
      for (int h = 0; h < hkv; ++h)
        for (int t = 0; t < qt; ++t) {
          const long long gkey = ((long long)r * hkv + h) * 100000 + t;
          if (suffix_readers[gkey] != 1) { printf("suffix read %d times\n", suffix_readers[gkey]); return 1; }
        }
    }
    for (const auto& kv : chunks)
      if ((int)kv.second.size() != nchunks[kv.first]) { printf("missing chunk index\n"); return 1; }
  }
  printf("ok: %d plans (%d fused), %lld items checked\n", iters, fused_plans, checked);
  return 0;
}
