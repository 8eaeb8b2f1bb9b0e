// gfx950 kernels of the acceptance walk of a verify tree, on the device.
//
// Replaces generation/d3_generator.py:204-225: starting with every candidate
// row valid, step a takes the first valid row, samples a token from the
// target's logits at that row's position a (model/utils.py:28-37), accepts
// it, and keeps only the rows whose draft token at position a + 1 equals it;
// the walk ends when no row is valid or the rows are exhausted.  The
// reference runs this loop on the host (nonzero(), sum() and a host-side list
// per step); here it is two launches with no host synchronisation, and its
// outputs feed the KV commit directly.
//
// Sampling.  At temperature 0 the token is torch.argmax (first index on
// ties).  At temperature T > 0 the reference draws torch.multinomial of
// softmax(logits / T), which torch computes as argmax(p / E), E ~ Exp(1)
// per token.  Here every node's token is drawn the same way in log space,
// argmax over tokens of x log2(e) - log2(E) with x = logits * (1/T) rounded
// to the logits dtype (torch's GPU division by a scalar), so no softmax pass
// is needed.  Each walk step visits a different node, so drawing all nodes'
// tokens up front and walking over them is the same process.  E = -ln(u),
// u uniform from Philox4x32-10 (Salmon et al., SC 2011) with counter
// (token / 4, node, step) and key seed; `step` is a device counter the walk
// advances, so every call, and every replay of a captured call, draws anew.
//
//   argmax_chunks_kernel  [N nodes] x [C chunks of the vocabulary]: the max
//                         score of each chunk as one 64-bit key
//                         (order-preserving float bits, then the complement
//                         of the index, so a larger key is a larger score or,
//                         on ties, a smaller index).  Greedy: HBM bound, N * V
//                         logits read once; sampling: one Philox call per
//                         four tokens and two log2 per token on top.
//   greedy_walk_kernel    one workgroup: every node's token from its C keys
//                         and the rows' node ids and draft tokens into LDS,
//                         then the walk in one wave from LDS.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "d2sd_internal.h"
#include "plan.h"

namespace d2sd {

__device__ __forceinline__ unsigned long long argmax_key(float v, unsigned idx) {
  const unsigned u = v == 0.f ? 0u : __float_as_uint(v);  // -0 ranks as +0 (equal logits)
  const unsigned ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned lo = __shfl_xor((unsigned)k, off), hi = __shfl_xor((unsigned)(k >> 32), off);
    k = max_u64(k, ((unsigned long long)hi << 32) | lo);
  }
  return k;
}

// Running argmax of one lane: the first logit, then strictly greater
// replaces, so among equal logits the lane keeps its first (smallest) index.
struct LaneMax {
  float v = -INFINITY;
  int i = -1;
  __device__ __forceinline__ void add(float x, int idx) {
    const bool gt = x > v || i < 0;
    v = gt ? x : v;
    i = gt ? idx : i;
  }
};

// Philox4x32-10: ten rounds of
// (c0, c1, c2, c3) <- (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)),
// the key bumped by the Weyl constants between rounds.
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, unsigned k0, unsigned k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const unsigned hi0 = __umulhi(0xD2511F53u, c.x), lo0 = 0xD2511F53u * c.x;
    const unsigned hi1 = __umulhi(0xCD9E8D57u, c.z), lo1 = 0xCD9E8D57u * c.z;
    c = uint4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// -log2(E), E = -ln(u), u = (2 (w >> 9) + 1) 2^-24 in (0, 1) (exact in fp32).
// For u >= 15/16, E comes from the series of -ln(1 - d), d = 1 - u exact, so
// the smallest E (the largest scores) keep their relative precision.
__device__ __forceinline__ float neg_log2_exp(unsigned w) {
  const float u = (float)((w >> 9) * 2u + 1u) * 0x1p-24f;
  const float d = (float)((0x7FFFFFu - (w >> 9)) * 2u + 1u) * 0x1p-24f;  // 1 - u
  float e;
  if (d <= 0.0625f) {
    // d + d^2/2 + ... + d^7/7: truncation below 2^-28 relative
    e = d * (1.f + d * (0.5f + d * (1.f / 3.f + d * (0.25f + d * (0.2f + d * (1.f / 6.f + d * (1.f / 7.f)))))));
  } else {
    e = -__builtin_amdgcn_logf(u) * 0.69314718055994531f;
  }
  return -__builtin_amdgcn_logf(e);
}

template <bool BF16>
__device__ __forceinline__ float logit_at(const void* row, int t) {
  return BF16 ? __uint_as_float((unsigned)((const uint16_t*)row)[t] << 16) : ((const float*)row)[t];
}

template <bool BF16>
__device__ __forceinline__ float scaled_logit(float l, float inv_t) {
  const float x = l * inv_t;
  if (!BF16) return x;
  unsigned u = __float_as_uint(x);  // round to nearest even bf16 (finite logits)
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  return __uint_as_float(u);
}

template <bool BF16, bool SAMPLE>
__global__ __launch_bounds__(256) void argmax_chunks_kernel(const AcceptParams p) {
  const int chunk = blockIdx.x, node = blockIdx.y;
  const int v0 = chunk * p.chunk_len, v1 = min(p.vocab, v0 + p.chunk_len);  // v0: a multiple of 8
  LaneMax m;
  if (SAMPLE) {
    // four tokens per Philox call: quads [v0 / 4, ceil(v1 / 4))
    const void* row = BF16 ? (const void*)((const uint16_t*)p.logits + (long long)node * p.logits_stride)
                           : (const void*)((const float*)p.logits + (long long)node * p.logits_stride);
    const unsigned long long step = (unsigned long long)*p.rng_step;
    const float kLog2e = 1.4426950408889634f;
    for (int qd = v0 / 4 + (int)threadIdx.x; 4 * qd < v1; qd += (int)blockDim.x) {
      const uint4 w = philox4x32_10(uint4{(unsigned)qd, (unsigned)node, (unsigned)step, (unsigned)(step >> 32)},
                                    p.seed_lo, p.seed_hi);
      const unsigned ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 4 * qd + e;
        if (t < v1) {
          const float x = scaled_logit<BF16>(logit_at<BF16>(row, t), p.inv_temperature);
          m.add(x * kLog2e + neg_log2_exp(ws[e]), t);
        }
      }
    }
  } else if (BF16) {
    const uint16_t* row = (const uint16_t*)p.logits + (long long)node * p.logits_stride;
    // 16-byte vectors of 8 logits over [v0, vend) when rows are 16-byte
    // aligned; then the rest one by one
    const bool aligned = p.logits_stride % 8 == 0 && ((uintptr_t)p.logits & 15) == 0;
    const int vend = aligned ? v0 + ((v1 - v0) & ~7) : v0;
    const int step = 8 * (int)blockDim.x;
    // eight vectors per lane in flight per round (one round for chunks of
    // up to 16 K logits)
    for (int v = v0 + 8 * (int)threadIdx.x; v < vend; v += 8 * step) {
      uint4 u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) u[j] = v + j * step < vend ? *(const uint4*)(row + v + j * step) : uint4{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (v + j * step >= vend) break;
        const unsigned w[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          m.add(__uint_as_float(w[e] << 16), v + j * step + 2 * e);
          m.add(__uint_as_float(w[e] & 0xFFFF0000u), v + j * step + 2 * e + 1);
        }
      }
    }
    for (int t = vend + (int)threadIdx.x; t < v1; t += (int)blockDim.x)
      m.add(__uint_as_float((unsigned)row[t] << 16), t);
  } else {
    const float* row = (const float*)p.logits + (long long)node * p.logits_stride;
    for (int t = v0 + (int)threadIdx.x; t < v1; t += (int)blockDim.x) m.add(row[t], t);
  }
  unsigned long long best = m.i < 0 ? 0ull : argmax_key(m.v, (unsigned)m.i);
  best = wave_max_u64(best);
  __shared__ unsigned long long wmax[4];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) wmax[wv] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = wmax[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) k = max_u64(k, wmax[i]);
    p.keys[(long long)node * p.chunks + chunk] = k;
  }
}

// The walk.  Phase 1 (all threads): each node's argmax from its chunk keys,
// and the rows' node ids and draft tokens, into LDS.  Phase 2 (wave 0, lane r
// owns candidate row r): the walk itself, from LDS only.
__global__ __launch_bounds__(256) void greedy_walk_kernel(const AcceptParams p) {
  __shared__ unsigned long long key_of[kAcceptMaxNodes];
  __shared__ int node_at[kAcceptMaxCells];
  __shared__ long long draft_at[kAcceptMaxCells];
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int nd = tid; nd < p.num_nodes; nd += nt) key_of[nd] = 0ull;
  __syncthreads();
  // the nodes' chunk keys, eight independent loads in flight per thread,
  // folded per node with LDS atomic maxima
  const int total = p.num_nodes * p.chunks;
  for (int base = tid; base < total; base += 8 * nt) {
    unsigned long long k[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) k[j] = base + j * nt < total ? p.keys[base + j * nt] : 0ull;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (base + j * nt < total)
        __hip_atomic_fetch_max(&key_of[(base + j * nt) / p.chunks], k[j], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  const int cells = p.num_rows * p.row_len;
  for (int c = tid; c < cells; c += nt) {
    node_at[c] = p.node_index[c];
    draft_at[c] = p.draft_ids[c];
  }
  __syncthreads();
  if (p.node_tokens)
    for (int nd = tid; nd < p.num_nodes; nd += nt)
      p.node_tokens[nd] = (long long)(0xFFFFFFFFu - (unsigned)key_of[nd]);
  if (tid == 0 && p.rng_step) p.rng_step[0] += 1;  // the chunk pass has read it
  if (tid >= 64) return;
  const int lane = tid;
  bool valid = lane < p.num_rows;
  int a = 0, vb = 0;
  while (true) {
    const unsigned long long vmask = __ballot(valid);
    if (vmask == 0ull) break;  // (only before the first step with num_rows == 0)
    vb = __ffsll((long long)vmask) - 1;  // first valid row
    const int node = node_at[vb * p.row_len + a];
    if (node < 0 || node >= p.num_nodes) break;  // not a node of the logits: the walk stops here
    const long long tok = (long long)(0xFFFFFFFFu - (unsigned)key_of[node]);
    if (lane == 0) {
      p.accept_ids[a] = tok;
      p.accept_nodes[a] = node;
    }
    ++a;
    if (a == p.row_len) break;
    if (valid) valid = draft_at[lane * p.row_len + a] == tok;
    if (__ballot(valid) == 0ull) break;
  }
  if (lane == 0) {
    p.result[0] = a;
    p.result[1] = vb;
  }
}

void greedy_accept_chunks(int num_nodes, int vocab, int& chunks, int& chunk_len) {
  // enough workgroups to cover the device (>= 2048 in total), chunks of at
  // least 1024 logits, chunk_len a multiple of 8
  const int want = std::max(1, (2048 + std::max(num_nodes, 1) - 1) / std::max(num_nodes, 1));
  const int c = std::max(1, std::min((vocab + 1023) / 1024, want));
  chunk_len = ((vocab + c - 1) / c + 7) & ~7;
  chunks = std::max(1, (vocab + chunk_len - 1) / chunk_len);
}

hipError_t launch_greedy_accept(const AcceptParams& p, bool bf16, hipStream_t s) {
  if (p.num_nodes <= 0) return hipSuccess;
  const dim3 grid((unsigned)p.chunks, (unsigned)p.num_nodes);
  const bool sample = p.rng_step != nullptr;
  if (sample) {
    if (bf16) hipLaunchKernelGGL((argmax_chunks_kernel<true, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((argmax_chunks_kernel<false, true>), grid, dim3(256), 0, s, p);
  } else {
    if (bf16) hipLaunchKernelGGL((argmax_chunks_kernel<true, false>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((argmax_chunks_kernel<false, false>), grid, dim3(256), 0, s, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(greedy_walk_kernel, dim3(1), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace d2sd
