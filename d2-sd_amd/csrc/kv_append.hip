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
// per layer (half the writes into fp8 pools).
//
// fp8 pools (OCP e4m3fn bytes holding value / scale[head], the format the
// cascade kernels dequantise): each value becomes e4m3fn(x / scale), the
// quotient correctly rounded in fp32, clamped to +-448 (the largest finite
// e4m3fn) and rounded to nearest even - torch's float -> float8_e4m3fn cast
// after a clamp (the cast alone turns |q| >= 480 into NaN); a NaN quotient
// becomes the e4m3fn NaN byte 0x7F with its sign, as torch's clamp and cast.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "d2sd_internal.h"
#include "plan.h"

namespace d2sd {

// e4m3fn byte of f, |f| <= 448: round to nearest even.  Below 2^-6 the
// format is subnormal with step 2^-9 (f * 512 rounded; 8 is the smallest
// normal, byte 0x08); above, the exponent is rebiased from 127 to 7 and the
// 20 dropped mantissa bits are rounded half to even.
__device__ __forceinline__ unsigned e4m3fn_byte(float f) {
  unsigned u = __float_as_uint(f);
  const unsigned sign = (u >> 24) & 0x80u;
  u &= 0x7FFFFFFFu;
  unsigned r;
  if (u < 0x3C800000u) {
    r = (unsigned)rintf(__uint_as_float(u) * 512.f);
  } else {
    u = u - 0x3C000000u + 0x7FFFFu + ((u >> 20) & 1u);
    r = u >> 20;
  }
  return r | sign;
}

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
  const bool fp8 = p.pool_dtype == KV_FP8;
  const float* kscale = fp8 ? (const float*)p.k_scale[layer] : nullptr;
  const float* vscale = fp8 ? (const float*)p.v_scale[layer] : nullptr;
  for (int c = threadIdx.x; c < 2 * nch; c += blockDim.x) {
    const bool is_v = c >= nch;
    const int cc = is_v ? c - nch : c;
    const int h = cc / cpr, d = 8 * (cc - h * cpr);
    const long long src = (long long)node * p.new_stride_n + (long long)h * p.new_stride_h + d;
    const long long dst = (long long)page * p.pool_stride_page + (long long)h * p.pool_stride_head +
                          (long long)slot * p.pool_stride_tok + d;
    const uint4 val = *(const uint4*)((is_v ? vnew : knew) + src);
    if (fp8) {
      // 8 values -> 8 e4m3fn bytes
      const float s = (is_v ? vscale : kscale)[h];
      const unsigned w[4] = {val.x, val.y, val.z, val.w};
      unsigned b[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned bits = ((w[e >> 1] >> (16 * (e & 1))) << 16) & 0xFFFF0000u;
        const float x = __uint_as_float(bits);
        const float qr = __fdiv_rn(x, s);
        const float q = fminf(fmaxf(qr, -448.f), 448.f);
        // a NaN quotient stays NaN (torch's clamp keeps it; the cast makes it
        // 0x7F with the NaN's sign: x's when x is NaN, else s's, else the
        // negative default NaN of 0/0 and inf/inf); fminf / fmaxf would
        // turn it into -448
        const unsigned nan_byte = 0x7Fu | ((isnan(x) ? bits : isnan(s) ? __float_as_uint(s) : 0x80000000u) >> 24 & 0x80u);
        b[e >> 2] |= (isnan(qr) ? nan_byte : e4m3fn_byte(q)) << (8 * (e & 3));
      }
      uint8_t* pool = (uint8_t*)(is_v ? p.v_pool[layer] : p.k_pool[layer]);
      *(uint2*)(pool + dst) = uint2{b[0], b[1]};
    } else {
      uint16_t* pool = (uint16_t*)(is_v ? p.v_pool[layer] : p.k_pool[layer]);
      *(uint4*)(pool + dst) = val;
    }
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
