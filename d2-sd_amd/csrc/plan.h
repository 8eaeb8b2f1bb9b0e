// Host-side work planners (plan.cpp) and kernel launchers.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>

#include <algorithm>
#include <vector>

#include "d2sd_internal.h"

namespace d2sd {

// ---- cascade verify attention (verify_attention.hip) ----
struct VerifyPlanInput {
  int num_reqs;
  const int* qo_indptr;          // host [num_reqs + 1]
  const int* prefix_len;         // host [num_reqs]
  const int* page_indptr;        // host [num_reqs + 1] (paged prefix)
  const int* prefix_tok_indptr;  // host [num_reqs] (contiguous prefix; nullable => 0)
  int num_qo_heads, num_kv_heads, head_dim;
  int window_left;
  int num_cus;
  int max_splits;  // 0: no limit beyond kMaxVerifySplits
  int waves;       // 0: choose; else 2, 4 or 8
  int page_size;   // 0: contiguous prefix
  // Two-segment contiguous prefix (nullable): keys [0, prefix_split[r]) of
  // request r are the first segment (prefix_tok_indptr), keys
  // [prefix_split[r], prefix_len[r]) the second (SRC_PREFIX2 items, token
  // prefix2_tok_indptr[r] + key - prefix_split[r]; nullable => 0).
  const int* prefix_split;
  const int* prefix2_tok_indptr;
};

struct VerifyPlanOutput {
  std::vector<VerifyItem> items;    // attention launch
  std::vector<VerifyMerge> merges;  // merge launch
  int waves;
  int rows;                         // rows per workgroup tile (= per partial slot)
  int num_slots;
  int max_splits_used;
  int num_groups;                   // (request, kv head, q-tile) groups
  int fused;                        // 1: no group is split; SRC_BOTH items, no partials, no merge
  size_t workspace_bytes;
};

int plan_verify(const VerifyPlanInput& in, VerifyPlanOutput& out);

// Pages that keys [b, e) of a pool with 2^log2_page keys per page span.
inline long long pages_spanned(long long b, long long e, int log2_page) {
  return e > b ? ((e - 1) >> log2_page) - (b >> log2_page) + 1 : 0;
}

// Longest prefix chunk (64-key tiles) whose page ids fit the kernel's LDS
// staging (kMaxStagedPages) for page size P (0: contiguous, no bound).  A
// dynamic plan's run-time chunk may start at any key and be up to 63 keys
// longer than planned (its boundaries are rescaled and rounded to 64 keys,
// the last one kept at the current length), so T tiles may read
// 64 T + 63 keys: that spans at most (64 T + 61 + P) / P pages, which stays
// <= kMaxStagedPages iff 64 T <= (kMaxStagedPages - 1) P - 62.
inline int verify_max_chunk_tiles(int page_size) {
  if (page_size <= 0) return 1 << 30;
  const long long t = ((long long)(kMaxStagedPages - 1) * page_size - 62) / 64;
  return (int)std::max<long long>(1, std::min<long long>(t, 1 << 30));
}
// Workgroups of the attention launch resident per CU (LDS bound) and packed
// rows per workgroup, by waves per workgroup (2: 64-row waves; 4, 8: 32-row
// waves).
int verify_wgs_per_cu(int waves);
int verify_rows(int waves);
int verify_auto_waves(const VerifyPlanInput& in, int num_cus);

// kind: KIND_SPLIT, KIND_FUSED (VerifyPlanOutput::fused), KIND_INPLACE or
// KIND_SEGMENTS (a plan with SRC_PREFIX2 items)
hipError_t launch_verify_attention(const VerifyParams& p, int head_dim, int waves, bool paged, bool fp8, int kind,
                                   int nitems, hipStream_t s);
hipError_t launch_verify_merge(const VerifyParams& p, int head_dim, int rows, int nmerges, hipStream_t s);
// Device address of this GPU's library-owned workspace (kVerifyScratchBytes).
hipError_t verify_scratch(void** ptr);

// ---- accepted-branch KV commit (kv_append.hip) ----
hipError_t launch_kv_append(const KvAppendParams& p, bool advance, hipStream_t s);

// ---- candidate-tree build (tree_build.hip) ----
hipError_t launch_d3_tree_build(const TreeBuildParams& p, hipStream_t s);

// ---- QK RMSNorm + RoPE (qk_rope.hip) ----
hipError_t launch_qk_norm_rope(const QkRopeParams& p, hipStream_t s);

// ---- greedy acceptance walk (accept.hip) ----
hipError_t launch_greedy_accept(const AcceptParams& p, bool bf16, hipStream_t s);
// vocabulary chunks per node of the argmax pass
void greedy_accept_chunks(int num_nodes, int vocab, int& chunks, int& chunk_len);

// ---- single-source drop-ins (attention.hip) ----
int choose_waves(int rows_per_head_max);
int blocks_per_cu(int waves);
void plan_single(int qo_len, int kv_len, int num_qo_heads, int num_kv_heads, int head_dim,
                 int window_left, int num_cus, ImplicitWork& imp, int& waves, size_t& workspace_bytes);

// src: 0 = p.src[0] (single source), 1 = p.src[1]
hipError_t launch_attention(const AttnParams& p, int head_dim, int waves, int src, bool fp8, bool paged,
                            bool masked, int nblocks, hipStream_t s);
hipError_t launch_merge(const AttnParams& p, int head_dim, int rows_per_tile, int nitems, hipStream_t s);
hipError_t launch_merge_state(void* v, long long v_sn, long long v_sh, float* s, long long s_sn,
                              const void* vo, long long vo_sn, long long vo_sh, const float* so,
                              long long so_sn, int n, int h, int d, int base2, hipStream_t stream);

}  // namespace d2sd
