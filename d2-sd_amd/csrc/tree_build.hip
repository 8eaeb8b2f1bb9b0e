// gfx950 kernel of the candidate-tree build of one D2SD step
// (generation/d3_generator.py:116-180), on the device:
//
//   rates[0] = 1 - c0; rates[k] = cumprod(c)[k-1] * (1 - c_k)       (:117-121)
//   boundaries = sorted(topk(rates, topk))                           (:123-125)
//   rows: the DFlash block (+ its continuation when block_size_2 >
//         block_size), then per boundary pl a row sharing the first pl + 1
//         tokens of the DFlash block                                  (:127-180)
//
// and from the rows the token tree the cascade kernels read: unique nodes,
// node_index [rows, block_size_2], parents and the packed ancestor mask, in a
// fixed capacity so that one captured graph serves every step (nodes past
// the tree's size are roots that see only themselves; rows past its row
// count repeat the DFlash row).  The reference does the top-k on the host
// (.tolist()); here nothing leaves the device.
//
// Arithmetic follows torch's GPU kernels for the dtype of the confidences
// (the draft's softmax probabilities): bf16 -> the cumulative product runs
// sequentially with every product rounded to bf16, 1 - c and the products
// round to bf16; fp32 -> fp32 throughout.  Equal rates are ranked by index.
//
// One wave: lane i < block_size - 1 owns boundary i; every node's ancestor
// set is two runs of node ids (the shared part of the DFlash row, then its
// own row's new nodes), so each mask word is computed independently.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "d2sd_internal.h"
#include "plan.h"

namespace d2sd {

namespace {

__device__ __forceinline__ float round_bf16(float x) {
  unsigned u = __float_as_uint(x);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  return __uint_as_float(u);
}

// bits [a, b] (inclusive) of 64-bit word w
__device__ __forceinline__ unsigned long long range_bits(int a, int b, int w) {
  const int lo = max(a, 64 * w), hi = min(b, 64 * w + 63);
  if (lo > hi) return 0ull;
  const int n = hi - lo + 1;
  const unsigned long long m = n == 64 ? ~0ull : ((1ull << n) - 1ull);
  return m << (lo - 64 * w);
}

}  // namespace

__global__ __launch_bounds__(64) void d3_tree_build_kernel(const TreeBuildParams p) {
  __shared__ float cum[64];
  __shared__ float rates[64];
  __shared__ int shared_len[kTreeMaxRows], base[kTreeMaxRows];
  __shared__ int nrows_s, nnodes_s;
  const int lane = threadIdx.x;
  const int n = p.block_size - 1;  // boundaries (<= 64)
  const int Lb = p.block_size_2;
  const bool bf = p.conf_bf16 != 0;
  auto rnd = [&](float x) { return bf ? round_bf16(x) : x; };

  float c = 0.f;
  if (lane < n) c = bf ? __uint_as_float((unsigned)((const uint16_t*)p.conf)[lane] << 16) : ((const float*)p.conf)[lane];
  // cumulative product, sequentially (lane 0), each product rounded
  if (lane < n) cum[lane] = c;
  __syncthreads();
  if (lane == 0) {
    float acc = 1.f;
    for (int i = 0; i < n; ++i) {
      acc = rnd(__fmul_rn(acc, cum[i]));
      cum[i] = acc;
    }
  }
  __syncthreads();
  float r = 0.f;
  if (lane < n) {
    const float om = rnd(1.f - c);
    r = lane == 0 ? om : rnd(__fmul_rn(cum[lane - 1], om));
    rates[lane] = r;
    if (p.rates) p.rates[lane] = r;
  }
  __syncthreads();
  // top-k: rank = boundaries with a larger rate, or an equal rate and a smaller index
  const int k = min(p.topk, n);
  bool sel = false;
  if (lane < n) {
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += (rates[j] > r || (rates[j] == r && j < lane)) ? 1 : 0;
    sel = rank < k && lane + 1 < Lb;  // a boundary whose anchor lies in the block (d3_generator.py:140-141)
  }
  const unsigned long long ballot = __ballot(sel);
  if (lane == 0) {
    // logical row 0 = the DFlash row; rows 1.. = the boundaries, increasing
    int rows = 1, nodes = Lb;
    shared_len[0] = Lb;
    base[0] = 0;
    for (unsigned long long b = ballot; b; b &= b - 1) {
      const int pl = __builtin_ctzll(b);
      shared_len[rows] = pl + 1;
      base[rows] = nodes;
      nodes += Lb - (pl + 1);
      ++rows;
    }
    nrows_s = rows;
    nnodes_s = nodes;
    *p.num_nodes = nodes;
    if (p.num_rows) *p.num_rows = rows;
  }
  __syncthreads();
  const int rows = nrows_s, nodes = nnodes_s;

  // output row of logical row j: with block_size_2 == block_size the DFlash
  // row comes last (d3_generator.py:174-175)
  const bool dflash_last = Lb == p.block_size;
  for (int o = 0; o < p.rows_cap; ++o) {
    int j = o;
    if (o >= rows) j = 0;                     // padding rows repeat the DFlash row
    else if (dflash_last) j = (o == rows - 1) ? 0 : o + 1;
    for (int pos = lane; pos < Lb; pos += 64)
      p.node_index[(long long)o * Lb + pos] = pos < shared_len[j] ? pos : base[j] + pos - shared_len[j];
    if (p.shared && lane == 0) p.shared[o] = shared_len[j];
  }
  // parents and ancestor masks, one node per lane
  for (int v = lane; v < p.capacity; v += 64) {
    int a0 = v, b0 = v, a1 = 1, b1 = 0, parent = -1;  // runs [a0, b0] and [a1, b1]
    if (v < Lb) {
      a0 = 0;
      parent = v - 1;
    } else if (v < nodes) {
      int j = 1;
      while (j + 1 < rows && v >= base[j + 1]) ++j;
      const int s = shared_len[j], pos = s + v - base[j];
      a0 = 0;
      b0 = s - 1;
      a1 = base[j];
      b1 = v;
      parent = v > base[j] ? v - 1 : pos - 1;
    }
    p.parents[v] = parent;
    for (int w = 0; w < p.mask_words; ++w)
      p.tree_mask[(long long)v * p.mask_words + w] = range_bits(a0, b0, w) | range_bits(a1, b1, w);
  }
}

hipError_t launch_d3_tree_build(const TreeBuildParams& p, hipStream_t s) {
  hipLaunchKernelGGL(d3_tree_build_kernel, dim3(1), dim3(64), 0, s, p);
  return hipGetLastError();
}

}  // namespace d2sd
