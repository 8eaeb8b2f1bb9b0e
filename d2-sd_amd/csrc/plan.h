// Host-side work planner interface (plan.cpp).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>

#include <vector>

#include "d2sd_internal.h"

namespace d2sd {

struct PlanInput {
  int num_reqs;
  const int* qo_indptr;   // host [num_reqs + 1]
  const int* prefix_len;  // host [num_reqs]
  int num_qo_heads, num_kv_heads, head_dim;
  int window_left;
  int num_cus;
  int max_splits;
  int waves;      // 0: choose
  int page_size;  // 0: contiguous prefix
};


struct PlanOutput {
  std::vector<WorkItem> prefix_work;  // prefix launch (split-KV partials)
  std::vector<WorkItem> suffix_work;  // suffix launch (tree attention + merge)
  int waves;
  int suffix_waves;
  int rows_per_tile;
  int num_slots;
  int max_splits_used;
  size_t workspace_bytes;
};

int choose_waves(int rows_per_head_max);
int blocks_per_cu(int waves);
int plan_cascade(const PlanInput& in, PlanOutput& out);
void plan_single(int qo_len, int kv_len, int num_qo_heads, int num_kv_heads, int head_dim,
                 int window_left, int num_cus, ImplicitWork& imp, int& waves, size_t& workspace_bytes);

// attention.hip launchers
// src: 0 = p.src[0] (prefix / single source), 1 = p.src[1] (suffix tree)
hipError_t launch_attention(const AttnParams& p, int head_dim, int waves, int src, bool fp8, bool paged,
                            bool masked, int nblocks, hipStream_t s);
hipError_t launch_merge(const AttnParams& p, int head_dim, int rows_per_tile, int nitems, hipStream_t s);
hipError_t launch_merge_state(void* v, long long v_sn, long long v_sh, float* s, long long s_sn,
                              const void* vo, long long vo_sn, long long vo_sh, const float* so,
                              long long so_sn, int n, int h, int d, int base2, hipStream_t stream);

}  // namespace d2sd
