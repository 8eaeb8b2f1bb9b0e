// gfx950 kernel: per-head RMSNorm of the new queries and keys followed by
// rotary position embedding, in place, in one launch.
//
// Replaces generation/verification.py:113-123 (Qwen3: attn.q_norm / k_norm,
// then the transposes and _apply_rotary_pos_emb_qwen3; GPT-OSS: RoPE only,
// _apply_rotary_pos_emb_gpt_oss) — about ten elementwise kernels and two
// layout copies per layer — for the node-major [tokens, heads, head_dim]
// layout the verify attention reads, so no transpose is needed at all.
//
// Numerics follow the reference's bf16 tensor ops step for step
// (transformers Qwen3RMSNorm and rotate_half RoPE):
//   h   = float(x) * (1 / sqrt(mean(float(x)^2) + eps))      fp32
//   y   = bf16(w * bf16(h))                                   (norm on)
//   out = bf16(bf16(y * cos) + bf16(rotate_half(y) * sin))
// with rotate_half(y)[i] = -y[i + D/2] (i < D/2), y[i - D/2] (i >= D/2) and
// cos/sin of D columns (Qwen3, halves equal) or D/2 columns (GPT-OSS).
//
// One wave per (token, head): lane l holds head dims l + 64 j (j < D / 64);
// the rotation partner of dim i is i +- D/2, in the same lane for D >= 128
// and in lane l ^ 32 for D = 64.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "d2sd_internal.h"
#include "plan.h"

namespace d2sd {

__device__ __forceinline__ float bf(uint16_t v) { return __uint_as_float((unsigned)v << 16); }

// round-to-nearest-even float -> bf16 (finite inputs)
__device__ __forceinline__ uint16_t to_bf(float f) {
  const unsigned u = __float_as_uint(f);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const QkRopeParams p) {
  constexpr int E = D / 64;  // dims per lane
  const int wave = (int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int heads = p.num_qo_heads + p.num_kv_heads;
  if (wave >= p.num_tokens * heads) return;
  const int t = wave / heads, h = wave - t * heads;
  const bool is_k = h >= p.num_qo_heads;
  uint16_t* x = (uint16_t*)(is_k ? p.k : p.q) + (long long)t * (is_k ? p.k_stride_n : p.q_stride_n) +
                (long long)(is_k ? h - p.num_qo_heads : h) * (is_k ? p.k_stride_h : p.q_stride_h);
  const uint16_t* w = (const uint16_t*)(is_k ? p.k_norm : p.q_norm);

  // every load up front, in one round (absent weights / tables read x as a
  // stand-in, never used)
  const uint16_t* cs = p.cos ? (const uint16_t*)p.cos + (long long)t * p.cs_stride : x;
  const uint16_t* sn = p.cos ? (const uint16_t*)p.sin + (long long)t * p.cs_stride : x;
  const uint16_t* wp = w ? w : x;
  float y[E], wv[E], cv[E], sv[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int d = lane + 64 * j;
    const int dc = p.cos && p.half_cos ? (d & (D / 2 - 1)) : d;
    y[j] = bf(x[d]);
    wv[j] = bf(wp[d]);
    cv[j] = bf(cs[dc]);
    sv[j] = bf(sn[dc]);
  }
  if (w) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < E; ++j) ss += y[j] * y[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    const float r = 1.0f / sqrtf(ss / (float)D + p.eps);
#pragma unroll
    for (int j = 0; j < E; ++j) y[j] = bf(to_bf(wv[j] * bf(to_bf(y[j] * r))));
  }
  if (p.cos) {
    float rot[E];
    if constexpr (D == 64) {
      const float other = __shfl_xor(y[0], 32);
      rot[0] = lane < 32 ? -other : other;
    } else {
#pragma unroll
      for (int j = 0; j < E; ++j) rot[j] = j < E / 2 ? -y[j + E / 2] : y[j - E / 2];
    }
    float out[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const float a = bf(to_bf(y[j] * cv[j]));
      const float b = bf(to_bf(rot[j] * sv[j]));
      out[j] = a + b;
    }
#pragma unroll
    for (int j = 0; j < E; ++j) y[j] = out[j];
  }
#pragma unroll
  for (int j = 0; j < E; ++j) x[lane + 64 * j] = to_bf(y[j]);
}

hipError_t launch_qk_norm_rope(const QkRopeParams& p, hipStream_t s) {
  const long long waves = (long long)p.num_tokens * (p.num_qo_heads + p.num_kv_heads);
  if (waves <= 0) return hipSuccess;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  switch (p.head_dim) {
    case 64: hipLaunchKernelGGL(qk_norm_rope_kernel<64>, grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL(qk_norm_rope_kernel<128>, grid, block, 0, s, p); break;
    case 256: hipLaunchKernelGGL(qk_norm_rope_kernel<256>, grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace d2sd
