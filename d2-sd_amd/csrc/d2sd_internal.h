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
};

enum : int { MASK_NONE = 0, MASK_CAUSAL = 1, MASK_TREE = 2 };

// Page ids one attention workgroup stages in LDS (its split's pages).
constexpr int kMaxStagedPages = 1024;
enum : int { KV_BF16 = 0, KV_FP8 = 1 };

// One attention workgroup of the single-source kernels: rows
// [qtile*ROWS, (qtile+1)*ROWS) of the packed (token, query-head) rows that read
// kv head `kvh` of request `req`, against keys [kv_begin, kv_end) of key
// source `src`, with epilogue `mode`.
struct WorkItem {
  int req, kvh, qtile, src, kv_begin, kv_end, slot, mode;
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

// Uniform work decomposition of the single-source kernels: every request
// has qo_len queries and kv_len keys; items are ordered so that all q-tiles
// reading one (request, kv head, split) key chunk land on the same XCD
// (workgroups are dealt to the 8 XCDs round-robin).
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
  const float* sinks;            // nullable, [Hq]
  KvSource src[2];
  ImplicitWork imp;
  float sm_scale;
  float sm_scale_log2;           // sm_scale * log2(e)
  int num_kv_heads;
  int group;                     // Hq / Hkv
  int lse_base2;
  int num_merge;
};


// ---------------------------------------------------------------------------
// Cascade verify attention (verify_attention.hip): one attention launch whose
// workgroups each own the packed rows of one (request, kv head, q-tile) group
// (32 per wave; 64 per wave of a two-wave workgroup) and either one key chunk
// of the shared prefix or the whole suffix tree, then one merge launch.
// ---------------------------------------------------------------------------
// Keys an item reads: a chunk of the shared prefix, the suffix tree,
// (SRC_BOTH) its group's whole visible prefix and then its suffix tree, or a
// chunk of the second segment of a two-segment contiguous prefix (kv_begin,
// kv_end and base in that segment's own key numbering).
enum : int { SRC_PREFIX = 0, SRC_SUFFIX = 1, SRC_BOTH = 2, SRC_PREFIX2 = 3 };

// Kinds of cascade plans (one attention-kernel instantiation each): split
// prefixes with partial states and a merge launch, fused (no split), in-place
// suffix items (the drop-in runner's per-row local level), and split plans
// over a two-segment contiguous prefix.
enum : int { KIND_SPLIT = 0, KIND_FUSED = 1, KIND_INPLACE = 2, KIND_SEGMENTS = 3 };

// 64 bytes; everything a workgroup needs is baked in by the planner so that
// the kernel's first dependent load is the item itself.
struct VerifyItem {
  int req, kvh, qtile, src;
  int kv_begin, kv_end;  // keys [kv_begin, kv_end) of the source (prefix: at the planned length)
  int slot;              // partial slot (MODE_PARTIAL)
  int mode;              // MODE_PARTIAL / MODE_FINAL / MODE_NOOP
  int q0, nq;            // the request's first query row and query count
  int base;              // paged: page_table index of the request's page 0;
                         // contiguous: token offset of the request's key 0
  int causal_off;        // MASK_CAUSAL: key j visible to query i iff j <= i + causal_off
  int kv0;               // prefix: first visible key at the planned length (window start)
  int plan_len;          // prefix: the request's planned prefix length
  int chunk;             // c | S << 16 for chunk c of the S chunks that split the request's
                         // whole visible prefix for this q-tile (dynamic plans re-partition
                         // it at the run-time length); 0: a piece of the prefix (dynamic
                         // plans scale its planned boundaries instead)
  int pad;
};

// First 64-key tile of chunk i of the S chunks that split nt tiles (a planned
// prefix, or a dynamic plan's run-time one): nt / S tiles each and one more
// for the first nt % S chunks.  The planner runs a group's first chunks
// in a CU's first round, each paired with a later chunk, so while a group's
// extra tiles fit its first-round chunks no CU holds two.  (constexpr: also
// compiled for the device.)
constexpr int dyn_chunk_start(int i, int S, int nt) {
  return i * (nt / S) + (i < nt % S ? i : nt % S);
}

// One 32-row block `blk` of a group whose partial slots
// [slot0, slot0 + nslots) are merged (nslots == 0: padding, no work).
struct VerifyMerge {
  int req, kvh, qtile, slot0, nslots, q0, nq, blk;
};

struct VerifySource {
  const void* k;
  const void* v;
  long long stride_tok, stride_head, stride_page;  // elements
  const int* page_table;   // nullable => contiguous
  const float* k_scale;    // fp8 dequant scale per kv head (nullable => 1)
  const float* v_scale;
  int log2_page;
  int fp8;
  int num_pages;           // paged: pages of the pool (page ids are clamped below it)
  int pad;
};

struct VerifyParams {
  const void* q;
  long long q_stride_n, q_stride_h;
  void* o;
  long long o_stride_n, o_stride_h;
  float* lse;              // nullable
  long long lse_stride_n;
  void* part_o;            // bf16 [slot][ROWS * D], register image
  float* part_lse;         // [slot][ROWS]
  const VerifyItem* items;
  const VerifyMerge* merges;
  const int* prefix_len;   // nullable: per-request prefix lengths read at run time (dynamic plans)
  const float* sinks;      // nullable, [Hq]
  const unsigned long long* tree_mask;  // [total_q][mask_words]
  VerifySource pre, suf;
  VerifySource pre2;       // second prefix segment (SRC_PREFIX2 items; contiguous)
  float sm_scale;
  float sm_scale_log2;
  int group;               // Hq / Hkv
  int mask_mode;           // suffix level: MASK_NONE / MASK_CAUSAL / MASK_TREE
  int mask_words;
  int lse_base2;
  int num_merges;
  int window_left;         // dynamic plans: the visible window (-1: whole prefix)
  int prefix_len_set;      // dynamic single-request plans: the current prefix length is
  int prefix_len_value;    //   prefix_len_value (a kernel argument) instead of prefix_len[0]
};

// Prefix key chunks per group are capped so that one merge batch holds all
// partials of a group (the chunks plus the suffix partial).
constexpr int kMaxVerifySplits = 15;

// Size of the library-owned workspace of d2sd_cascade_run_noalloc (per GPU).
constexpr unsigned long long kVerifyScratchBytes = 32ull << 20;

// ---------------------------------------------------------------------------
// Accepted-branch KV commit (kv_append.hip).
// ---------------------------------------------------------------------------
struct KvAppendParams {
  const int* node_ids;     // [num_accepted] rows of k_new / v_new, in cache order
  const int* page_table;   // the request's pages
  const uint64_t* k_new;   // [num_layers] addresses of bf16 [rows, Hkv, D]
  const uint64_t* v_new;
  const uint64_t* k_pool;  // [num_layers] addresses of the bf16 page pools
  const uint64_t* v_pool;
  long long new_stride_n, new_stride_h;                          // elements
  long long pool_stride_page, pool_stride_head, pool_stride_tok;  // elements
  int num_layers, num_kv_heads, head_dim;
  int log2_page;
  int prefix_len, num_accepted;
  int num_rows;    // rows of k_new / v_new (node ids outside are skipped)
  int pool_pages;  // pages of each pool (page ids outside are skipped)
  const int* num_accepted_dev;  // nullable: the count is read here (clamped to [0, num_accepted])
  int* prefix_len_dev;          // nullable: the cache length is read here
  int page_table_len;           // entries of page_table (device lengths are range-checked against it)
  int pool_dtype;               // KV_BF16 or KV_FP8 (e4m3fn bytes, value / scale)
  const uint64_t* k_scale;      // KV_FP8: [num_layers] addresses of fp32 [Hkv]
  const uint64_t* v_scale;
};

// ---------------------------------------------------------------------------
// Greedy acceptance walk (accept.hip).
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// QK RMSNorm + RoPE (qk_rope.hip).
// ---------------------------------------------------------------------------
struct QkRopeParams {
  void* q;                  // bf16 [tokens, Hq, D], head_dim contiguous (in place)
  void* k;                  // bf16 [tokens, Hkv, D]
  long long q_stride_n, q_stride_h, k_stride_n, k_stride_h;  // elements
  const void* q_norm;       // bf16 [D] RMSNorm weights (nullable: no norm)
  const void* k_norm;
  const void* cos;          // bf16 [tokens, D or D/2] (nullable: no rotation)
  const void* sin;
  long long cs_stride;      // elements between tokens of cos / sin
  float eps;
  int num_tokens, num_qo_heads, num_kv_heads, head_dim;
  int half_cos;             // cos / sin hold D/2 columns
};

// ---------------------------------------------------------------------------
// Candidate-tree build (tree_build.hip).
// ---------------------------------------------------------------------------
constexpr int kTreeMaxRows = 65;  // DFlash row + at most 64 boundaries
struct TreeBuildParams {
  const void* conf;          // [block_size - 1] bf16 or fp32
  int conf_bf16;
  int block_size, block_size_2, topk;
  int capacity;              // nodes of parents / tree_mask
  int rows_cap;              // rows of node_index / shared
  int mask_words;
  int* num_nodes;            // [1]
  int* num_rows;             // [1] nullable
  int* parents;              // [capacity]
  int* node_index;           // [rows_cap, block_size_2]
  unsigned long long* tree_mask;  // [capacity, mask_words]
  int* shared;               // [rows_cap] nullable
  float* rates;              // [block_size - 1] nullable
};

constexpr int kAcceptMaxNodes = 4096;  // logits rows of one walk
constexpr int kAcceptMaxCells = 2048;  // candidate rows x positions
struct AcceptParams {
  const void* logits;             // [num_nodes, vocab] bf16 or fp32, row stride logits_stride
  long long logits_stride;        // elements
  const int* node_index;          // [num_rows, row_len]
  const long long* draft_ids;     // [num_rows, row_len]
  long long* accept_ids;          // out [row_len]
  int* accept_nodes;              // out [row_len]
  int* result;                    // out [2]: acceptance length, final valid row
  unsigned long long* keys;       // workspace [num_nodes, chunks]
  int num_rows, row_len, num_nodes, vocab;
  int chunks, chunk_len;          // vocabulary chunks per node (chunk_len a multiple of 8)
  // sampling (temperature > 0): each node's token is the argmax of
  // x log2(e) - log2(E), x = logits * inv_temperature rounded to the logits
  // dtype, E = -ln(u), u from Philox4x32-10 with counter
  // (token / 4, node, step) and key seed
  float inv_temperature;
  unsigned seed_lo, seed_hi;
  long long* rng_step;            // [1] the step counter; the walk advances it by one
  long long* node_tokens;         // out [num_nodes] nullable: every node's token
};

}  // namespace d2sd
