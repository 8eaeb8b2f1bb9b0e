// gfx950 kernel of the accepted-branch KV commit: every layer's accepted
// tree nodes are written into the paged prefix cache in place, in one launch.
//
// Replaces generation/d3_generator.py:227-232, where each layer's cache grows
// by `torch.cat([layer.keys, k_win], dim=2)` (k_win = the accepted row's first
// acceptance_length new keys; likewise values): a copy of the whole cache per
// layer and step.  Here the new tokens land in pages the caller reserved, so
// the prefix stays where it is and one hipGraph can replay across steps.
//
// Work: block (i, layer) copies accepted token i of one layer: K and V rows of
// Hkv x D bf16 (2 KB each at Hkv 8, D 128), 16 bytes per lane.  Pure data
// movement, HBM bound: 2 * num_accepted * Hkv * D * 2 bytes read and written
// per layer.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "d2sd_internal.h"
#include "plan.h"

namespace d2sd {

__global__ __launch_bounds__(256) void kv_append_kernel(const KvAppendParams p) {
  const int i = blockIdx.x, layer = blockIdx.y;
  if (p.num_accepted_dev && i >= min(max(*p.num_accepted_dev, 0), p.num_accepted)) return;
  const int node = p.node_ids[i];
  if (node < 0 || node >= p.num_rows) return;  // not a row of k_new / v_new: nothing written
  const int L = p.prefix_len_dev ? *p.prefix_len_dev : p.prefix_len;
  if (L < 0) return;
  const int t = L + i;  // cache position of the token
  if ((t >> p.log2_page) >= p.page_table_len) return;  // no page reserved for it
  const int page = p.page_table[t >> p.log2_page];
  if (page < 0 || page >= p.pool_pages) return;
  const int slot = t & ((1 << p.log2_page) - 1);
  const int cpr = p.head_dim / 8;  // 16-byte chunks per head row
  const int nch = p.num_kv_heads * cpr;
  const uint16_t* knew = (const uint16_t*)p.k_new[layer];
  const uint16_t* vnew = (const uint16_t*)p.v_new[layer];
  uint16_t* kpool = (uint16_t*)p.k_pool[layer];
  uint16_t* vpool = (uint16_t*)p.v_pool[layer];
  for (int c = threadIdx.x; c < 2 * nch; c += blockDim.x) {
    const bool is_v = c >= nch;
    const int cc = is_v ? c - nch : c;
    const int h = cc / cpr, d = 8 * (cc - h * cpr);
    const long long src = (long long)node * p.new_stride_n + (long long)h * p.new_stride_h + d;
    const long long dst = (long long)page * p.pool_stride_page + (long long)h * p.pool_stride_head +
                          (long long)slot * p.pool_stride_tok + d;
    const uint4 val = *(const uint4*)((is_v ? vnew : knew) + src);
    *(uint4*)((is_v ? vpool : kpool) + dst) = val;
  }
}

// After the commit: the device cache length grows by the accepted count (a
// launch of its own, so that every block of the commit read the old length).
__global__ void advance_prefix_kernel(int* prefix_len, const int* num_accepted_dev, int num_accepted) {
  if (threadIdx.x == 0)
    *prefix_len += num_accepted_dev ? min(max(*num_accepted_dev, 0), num_accepted) : num_accepted;
}

hipError_t launch_kv_append(const KvAppendParams& p, bool advance, hipStream_t s) {
  if (p.num_accepted <= 0 || p.num_layers <= 0) return hipSuccess;
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)p.num_accepted, (unsigned)p.num_layers), dim3(256), 0, s, p);
  if (advance && p.prefix_len_dev)
    hipLaunchKernelGGL(advance_prefix_kernel, dim3(1), dim3(64), 0, s, p.prefix_len_dev, p.num_accepted_dev,
                       p.num_accepted);
  return hipGetLastError();
}

}  // namespace d2sd
