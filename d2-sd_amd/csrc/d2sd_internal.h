// Internal types shared by the gfx950 kernels (attention.hip), the host-side
// work planner (plan.cpp) and the C ABI (capi.cpp).
#pragma once

#include <stdint.h>

namespace d2sd {

// Epilogue of one attention workgroup.
enum : int {
  MODE_PARTIAL = 0,  // write fp32 (O, LSE) of its key chunk to a workspace slot
  MODE_FINAL = 1,    // only producer for its rows: write bf16 O and LSE directly
  MODE_INPLACE = 2,  // merge into the (O, LSE) already stored at the output
  MODE_NOOP = 3,     // padding item, exits immediately
  MODE_MERGE_SLOTS = 4,  // merge (mode >> 8) prefix partials at `slot` with its own state
};

enum : int { MASK_NONE = 0, MASK_CAUSAL = 1, MASK_TREE = 2 };

// Page ids one attention workgroup stages in LDS (its split's pages).
constexpr int kMaxStagedPages = 1024;
// Waves of the suffix (tree attention + merge) launch: 64-row blocks.
constexpr int kSuffixWaves = 2;
enum : int { KV_BF16 = 0, KV_FP8 = 1 };

// One attention workgroup: rows [qtile*ROWS, (qtile+1)*ROWS) of the packed
// (token, query-head) rows that read kv head `kvh` of request `req`, against
// keys [kv_begin, kv_end) of key source `src`.  `mode` holds the epilogue in
// its low 8 bits and, for MODE_MERGE_SLOTS, the partial count above them.
struct WorkItem {
  int req, kvh, qtile, src, kv_begin, kv_end, slot, mode;
};

// One merge item: rows of tile (req, kvh, qtile), partial slots
// [slot_begin, slot_begin + nslots), epilogue FINAL or INPLACE.
struct MergeItem {
  int req, kvh, qtile, slot_begin, nslots, mode, pad0, pad1;
};

// Where the keys/values of one level live.  Offsets are in elements.
struct KvSource {
  const void* k;
  const void* v;
  long long stride_tok;    // between consecutive tokens (inside a page)
  long long stride_head;   // between kv heads
  long long stride_page;   // between pages (paged only)
  long long stride_req;    // contiguous: per-request base (implicit work)
  const int* tok_indptr;   // contiguous: first token of each request (nullable)
  const int* page_indptr;  // paged: first page_table slot of each request
  const int* page_table;   // nullable => contiguous
  const int* kv_len;       // per-request key count (causal alignment; nullable)
  const unsigned long long* tree_mask;  // rows indexed like queries
  const float* k_scale;    // fp8 dequant scale per kv head (nullable => 1)
  const float* v_scale;
  int log2_page;
  int mask_mode;
  int mask_words;
  int dtype;               // KV_BF16 / KV_FP8
};

// Uniform work decomposition used when no explicit work list is given:
// every request has qo_len queries and kv_len keys; items are ordered so that
// all q-tiles reading one (request, kv head, split) key chunk land on the
// same XCD (workgroups are dealt to the 8 XCDs round-robin).
struct ImplicitWork {
  int num_reqs;
  int qtiles;
  int splits;
  int chunk_keys;   // keys per split (multiple of 64)
  int qo_len;
  int kv_len;
  int kv_begin;     // first visible key (window)
  int single_mode;  // epilogue when splits == 1 (FINAL or INPLACE)
};

struct AttnParams {
  const void* q;
  long long q_stride_n, q_stride_h, q_stride_req;
  const int* qo_indptr;          // nullable => request r starts at 0 (+q_stride_req)
  void* o;
  long long o_stride_n, o_stride_h, o_stride_req;
  float* lse;
  long long lse_stride_n, lse_stride_req;
  void* part_o;                  // bf16 [slot][ROWS * D], register image
  float* part_lse;               // [slot][ROWS]
  const WorkItem* work;          // nullable => implicit
  const MergeItem* merge;        // nullable => implicit
  const float* sinks;            // nullable, [Hq]
  KvSource src[2];
  ImplicitWork imp;
  float sm_scale;
  float sm_scale_log2;           // sm_scale * log2(e)
  int num_kv_heads;
  int group;                     // Hq / Hkv
  int lse_base2;
  int num_merge;
  int prefix_rows;               // rows per partial slot (MODE_MERGE_SLOTS)
};

}  // namespace d2sd
