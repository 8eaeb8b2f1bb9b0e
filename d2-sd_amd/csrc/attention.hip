// gfx950 (CDNA4) kernels for cascade tree-verification attention.
//
//   attn_kernel     GQA-packed split-KV attention over one key source (the
//                   shared prefix — contiguous or paged, bf16 or fp8 — or the
//                   suffix tree), with a partial / final / in-place-merge
//                   epilogue.  Replaces flashinfer.single_prefill_with_kv_cache
//                   (generation/verification.py:145-162, model/cascade_graph.py:54-57).
//   merge_kernel    log-sum-exp merge of split partials (+ optional merge into
//                   an existing state and the GPT-OSS sink rescale of
//                   generation/verification.py:173-176).
//   merge_state_kernel  flashinfer.merge_state_in_place
//                   (generation/verification.py:163-165, model/cascade_graph.py:58-60).
//
// Work decomposition.  The rows of one (request, kv head) are the packed
// (token n, query head j) pairs, row = n*g + j, so all g query heads that
// share a kv head ride in the same MFMA tile and each key/value element
// fetched from HBM feeds N*g query rows.  A workgroup of W waves owns
// ROWS = 32*W rows and a chunk of keys; each wave owns 32 rows.
//
// Per 64-key tile a wave computes S^T = K . Q^T with
// v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = its Q rows held in
// registers for the whole loop), so lane l holds the scores of ONE query
// row (l % 32) for 32 keys: the softmax max / sum are in-lane plus one
// exchange with lane l^32.  P^T is fed back as the B operand of
// O^T += V^T . P^T straight from those registers; V^T is staged in LDS with
// the key order inside every 16-key group permuted so that the A operand a
// lane reads matches the key order of the P^T values it already holds.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "d2sd_internal.h"

namespace d2sd {

typedef __bf16 bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Lazy rescaling: the running max used for exponentiation may trail the true
// row max by up to 2^kRescaleSlack before O and l are rescaled.
constexpr float kRescaleSlack = 8.0f;

__device__ __forceinline__ bf16x8 zero_bf16x8() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(bf16x8, z);
}

__device__ __forceinline__ unsigned pack_bf16x2(float a, float b) {
  f32x2 v = {a, b};
  return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ float bf16_lo(unsigned w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(unsigned w) { return __uint_as_float(w & 0xffff0000u); }

// ---------------------------------------------------------------------------
// Work items
// ---------------------------------------------------------------------------
__device__ __forceinline__ WorkItem implicit_work(const AttnParams& p, int b) {
  const ImplicitWork& im = p.imp;
  const int Q = im.qtiles;
  const int G = im.num_reqs * p.num_kv_heads * im.splits;
  int gidx, qt;
  if ((G & 7) == 0) {
    // Keep the q-tiles of one key chunk on one XCD (b % 8) so that the chunk
    // is fetched from HBM once and re-read from that XCD's L2.
    const int x = b & 7, k = b >> 3;
    gidx = x + 8 * (k / Q);
    qt = k % Q;
  } else {
    gidx = b / Q;
    qt = b % Q;
  }
  WorkItem w;
  const int split = gidx % im.splits;
  const int rest = gidx / im.splits;
  w.qtile = qt;
  w.kvh = rest % p.num_kv_heads;
  w.req = rest / p.num_kv_heads;
  w.src = 0;
  w.kv_begin = im.kv_begin + split * im.chunk_keys;
  w.kv_end = min(im.kv_len, w.kv_begin + im.chunk_keys);
  w.slot = ((w.req * p.num_kv_heads + w.kvh) * Q + qt) * im.splits + split;
  w.mode = im.splits > 1 ? MODE_PARTIAL : im.single_mode;
  return w;
}

__device__ __forceinline__ long long tok_offset(const KvSource& s, int req, int t) {
  if (s.page_table != nullptr) {
    const int pg = s.page_table[s.page_indptr[req] + (t >> s.log2_page)];
    return (long long)pg * s.stride_page + (long long)(t & ((1 << s.log2_page) - 1)) * s.stride_tok;
  }
  const int base = s.tok_indptr ? s.tok_indptr[req] : 0;
  return (long long)req * s.stride_req + (long long)(base + t) * s.stride_tok;
}

// fp8 e4m3fn (OCP) -> bf16, exact.  Bytes b0..b3 of w -> 4 bf16 in a u32x2.
__device__ __forceinline__ u32x2 fp8x4_to_bf16x4(unsigned w) {
  // e4m3fn placed in the top of an fp16: value(fp16) * 2^8 == value(e4m3fn)
  // for normals and subnormals alike (exponent bias 15 vs 7).  The 2^8 is
  // folded into the dequantisation scale by the caller.
  u32x2 r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const unsigned b0 = (w >> (16 * h)) & 0xffu, b1 = (w >> (16 * h + 8)) & 0xffu;
    const unsigned h0 = ((b0 & 0x80u) << 8) | ((b0 & 0x7fu) << 7);
    const unsigned h1 = ((b1 & 0x80u) << 8) | ((b1 & 0x7fu) << 7);
    const float f0 = (float)__builtin_bit_cast(_Float16, (unsigned short)h0);
    const float f1 = (float)__builtin_bit_cast(_Float16, (unsigned short)h1);
    // fp16 values with a 3-bit mantissa are exact in bf16: truncate.
    r[h] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
  }
  return r;
}

// ---------------------------------------------------------------------------
// Output epilogue shared by attn_kernel (FINAL / INPLACE) and merge_kernel.
// o4 holds 4 consecutive head-dim values (already normalised), lse is natural.
// ---------------------------------------------------------------------------
struct RowOut {
  bf16_t* o;     // row base (head-dim 0)
  float* lse;    // lse slot of this (token, head), nullable
};

__device__ __forceinline__ float load_lse_nat(const float* lse, int base2) {
  const float v = *lse;
  return base2 ? v * kLn2 : v;
}

// ---------------------------------------------------------------------------
// Attention kernel
// ---------------------------------------------------------------------------
template <int D, int W, bool FP8>
__global__ __launch_bounds__(64 * W) void attn_kernel(const AttnParams p) {
  constexpr int ROWS = 32 * W;
  constexpr int NT = 64 * W;
  constexpr int KP = D + 8;   // K tile pitch (elements)
  constexpr int VP = 64 + 8;  // V^T tile pitch (elements)
  constexpr int KCH = D / 8;  // 16-byte chunks per key row (bf16)
  constexpr int NK = 64 * KCH / NT;  // K chunks per thread == V keys per thread
  constexpr int VKG = 64 / NK;       // V key groups per d-chunk
  static_assert(NK >= 1 && NK <= 4, "tile/thread mismatch");

  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][64 * KP];
  __shared__ __attribute__((aligned(16))) bf16_t Vt[2][D * VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  const WorkItem w = p.work ? p.work[blockIdx.x] : implicit_work(p, blockIdx.x);
  if (w.mode == MODE_NOOP) return;
  const KvSource S = w.src ? p.src[1] : p.src[0];
  const bool fp8 = FP8 && (S.dtype == KV_FP8);

  const int g = p.group;
  const int q0 = p.qo_indptr ? p.qo_indptr[w.req] : 0;
  const int nq = p.qo_indptr ? p.qo_indptr[w.req + 1] - q0 : p.imp.qo_len;
  const int R = nq * g;
  const int row = w.qtile * ROWS + wv * 32 + l32;
  const bool rvalid = row < R;
  const int n = rvalid ? row / g : 0;
  const int j = rvalid ? row - n * g : 0;
  const int qh = w.kvh * g + j;

  // Q fragments (B operand of S^T = K Q^T): lane holds 8 consecutive head
  // dims at offset 8*hh of every 16-wide k step, for query row `row`.
  bf16x8 qf[D / 16];
  {
    const bf16_t* qp = (const bf16_t*)p.q + (long long)w.req * p.q_stride_req +
                       (long long)(q0 + n) * p.q_stride_n + (long long)qh * p.q_stride_h + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
      qf[ks] = rvalid ? *(const bf16x8*)(qp + 16 * ks) : zero_bf16x8();
  }

  float kscale = 1.f, vscale = 1.f;
  if (fp8) {
    kscale = (S.k_scale ? S.k_scale[w.kvh] : 1.f) * 256.f;
    vscale = (S.v_scale ? S.v_scale[w.kvh] : 1.f) * 256.f;
  }
  const float c = p.sm_scale_log2 * kscale;  // raw score -> log2 domain
  const float cn = p.sm_scale * kscale;      // raw score -> natural domain

  const int kv_begin = w.kv_begin, kv_end = w.kv_end;
  const int ntiles = (kv_end - kv_begin + 63) >> 6;
  const long long head_off = (long long)w.kvh * S.stride_head;
  const int mask_mode = S.mask_mode;
  const int kvlen_req = S.kv_len ? S.kv_len[w.req] : (p.work ? nq : p.imp.kv_len);
  const int causal_off = kvlen_req - nq;  // key j visible iff j <= i + causal_off
  const unsigned long long* mrow =
      (mask_mode == MASK_TREE && rvalid) ? S.tree_mask + (long long)(q0 + n) * S.mask_words : nullptr;

  // ---- global -> register tile loads ----
  u32x4 kr[NK], vr[NK];
  auto load_tile = [&](int kb) {
    const bf16_t* kbase = (const bf16_t*)S.k;
    const bf16_t* vbase = (const bf16_t*)S.v;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int c_ = tid + i * NT;
      const int key = c_ / KCH, dc = c_ % KCH;
      const int t = kb + key;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (t < kv_end) {
        const long long off = tok_offset(S, w.req, t) + head_off + dc * 8;
        if (fp8) {
          const u32x2 raw = *(const u32x2*)((const unsigned char*)S.k + off);
          const u32x2 lo = fp8x4_to_bf16x4(raw[0]), hi = fp8x4_to_bf16x4(raw[1]);
          val = (u32x4){lo[0], lo[1], hi[0], hi[1]};
        } else {
          val = *(const u32x4*)(kbase + off);
        }
      }
      kr[i] = val;
    }
    const int kg = tid % VKG, dc = tid / VKG;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int t = kb + kg * NK + i;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (t < kv_end) {
        const long long off = tok_offset(S, w.req, t) + head_off + dc * 8;
        if (fp8) {
          const u32x2 raw = *(const u32x2*)((const unsigned char*)S.v + off);
          const u32x2 lo = fp8x4_to_bf16x4(raw[0]), hi = fp8x4_to_bf16x4(raw[1]);
          val = (u32x4){lo[0], lo[1], hi[0], hi[1]};
        } else {
          val = *(const u32x4*)(vbase + off);
        }
      }
      vr[i] = val;
    }
  };

  // ---- register -> LDS (K row-major, V transposed with permuted key slots) ----
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int c_ = tid + i * NT;
      const int key = c_ / KCH, dc = c_ % KCH;
      *(u32x4*)(&Ks[buf][key * KP + dc * 8]) = kr[i];
    }
    const int kg = tid % VKG, dc = tid / VKG;
    const int kk = kg * NK;  // first key of this thread (NK consecutive keys)
    // slot of key kk inside its 16-key group: keys 4h+{0..3} and 4h+8+{0..3}
    // of half h are stored at slots 8h..8h+7 (the order in which a lane of
    // half h holds them in the S^T accumulator).
    const int slot = (kk & ~15) + 8 * ((kk >> 2) & 1) + (kk & 3) + 4 * ((kk >> 3) & 1);
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      bf16_t* dst = &Vt[buf][(dc * 8 + dd) * VP + slot];
      const int wi = dd >> 1;
      const int sh = (dd & 1) * 16;
      if constexpr (NK == 4) {
        const unsigned e0 = (vr[0][wi] >> sh) & 0xffffu, e1 = (vr[1][wi] >> sh) & 0xffffu;
        const unsigned e2 = (vr[2][wi] >> sh) & 0xffffu, e3 = (vr[3][wi] >> sh) & 0xffffu;
        *(u32x2*)dst = (u32x2){e0 | (e1 << 16), e2 | (e3 << 16)};
      } else if constexpr (NK == 2) {
        const unsigned e0 = (vr[0][wi] >> sh) & 0xffffu, e1 = (vr[1][wi] >> sh) & 0xffffu;
        *(unsigned*)dst = e0 | (e1 << 16);
      } else {
        *(unsigned short*)dst = (unsigned short)((vr[0][wi] >> sh) & 0xffffu);
      }
    }
  };

  f32x16 o[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mt][r] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;

  if (ntiles > 0) {
    load_tile(kv_begin);
    store_tile(0);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int buf = it & 1;
    const int kb = kv_begin + it * 64;
    if (it + 1 < ntiles) load_tile(kb + 64);

    // ---- S^T = K Q^T : two 32-key tiles ----
    f32x16 s0, s1;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s0[r] = 0.f; s1[r] = 0.f; }
    {
      const bf16_t* ka = &Ks[buf][l32 * KP + 8 * hh];
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const bf16x8 a0 = *(const bf16x8*)(ka + 16 * ks);
        const bf16x8 a1 = *(const bf16x8*)(ka + 32 * KP + 16 * ks);
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[ks], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[ks], s1, 0, 0, 0);
      }
    }

    // ---- masking ----
    // register r of 32-key tile kt holds key 32*kt + 8*(r/4) + 4*hh + r%4.
    const bool tail = kb + 64 > kv_end;
    if (tail || mask_mode != MASK_NONE) {
      unsigned long long mw = ~0ull;
      if (mask_mode == MASK_TREE) mw = mrow ? mrow[kb >> 6] : 0ull;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk0 = 8 * (r >> 2) + 4 * hh + (r & 3);
        const int kk1 = kk0 + 32;
        const int t0 = kb + kk0, t1 = kb + kk1;
        bool v0 = t0 < kv_end, v1 = t1 < kv_end;
        if (mask_mode == MASK_CAUSAL) {
          v0 = v0 && (t0 <= n + causal_off);
          v1 = v1 && (t1 <= n + causal_off);
        } else if (mask_mode == MASK_TREE) {
          v0 = v0 && ((mw >> kk0) & 1ull);
          v1 = v1 && ((mw >> kk1) & 1ull);
        }
        if (!v0) s0[r] = -INFINITY;
        if (!v1) s1[r] = -INFINITY;
      }
    }

    // ---- online softmax (lane-local row, partner lane l^32) ----
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const bool grow = (mx > m_run) && ((m_run == -INFINITY) || (mx - m_run) * c > kRescaleSlack);
    if (__any(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = (m_run == -INFINITY) ? 0.f : exp2f((m_run - m_new) * c);
      l_run *= alpha;
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;
      m_run = m_new;
    }
    const float mc = (m_run == -INFINITY) ? 0.f : m_run * c;
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = __builtin_amdgcn_exp2f(fmaf(s0[r], c, -mc));
      s1[r] = __builtin_amdgcn_exp2f(fmaf(s1[r], c, -mc));
      lsum += s0[r] + s1[r];
    }
    l_run += lsum;

    // ---- O^T += V^T P^T ----
    bf16x8 pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const f32x16& sv = (ks < 2) ? s0 : s1;
      const int base = 8 * (ks & 1);
      u32x4 u;
      u[0] = pack_bf16x2(sv[base + 0], sv[base + 1]);
      u[1] = pack_bf16x2(sv[base + 2], sv[base + 3]);
      u[2] = pack_bf16x2(sv[base + 4], sv[base + 5]);
      u[3] = pack_bf16x2(sv[base + 6], sv[base + 7]);
      pb[ks] = __builtin_bit_cast(bf16x8, u);
    }
    {
      const bf16_t* va = &Vt[buf][l32 * VP + 8 * hh];
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 a = *(const bf16x8*)(va + 32 * mt * VP + 16 * ks);
          o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ks], o[mt], 0, 0, 0);
        }
    }

    if (it + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const bool nonempty = l_tot > 0.f;
  const float inv = nonempty ? vscale / l_tot : 0.f;
  const float lse = nonempty ? m_run * cn + logf(l_tot) : -INFINITY;

  if (w.mode == MODE_PARTIAL) {
    const long long prow = (long long)w.slot * ROWS + wv * 32 + l32;
    float* po = p.part_o + prow * D;
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        f32x4 v = {o[mt][4 * q4] * inv, o[mt][4 * q4 + 1] * inv, o[mt][4 * q4 + 2] * inv,
                   o[mt][4 * q4 + 3] * inv};
        *(f32x4*)(po + 32 * mt + 8 * q4 + 4 * hh) = v;
      }
    if (hh == 0) p.part_lse[prow] = lse;
    return;
  }
  if (!rvalid) return;

  // FINAL / INPLACE: merge with the stored state if asked, then sink.
  bf16_t* orow = (bf16_t*)p.o + (long long)w.req * p.o_stride_req + (long long)(q0 + n) * p.o_stride_n +
                 (long long)qh * p.o_stride_h;
  float* lrow = p.lse ? p.lse + (long long)w.req * p.lse_stride_req + (long long)(q0 + n) * p.lse_stride_n + qh
                      : nullptr;
  float wa = 0.f, wb = 1.f, lse_out = lse;
  if (w.mode == MODE_INPLACE) {
    const float lo = load_lse_nat(lrow, p.lse_base2);
    const float m = fmaxf(lo, lse);
    if (m == -INFINITY) {
      wa = 1.f; wb = 0.f; lse_out = -INFINITY;
    } else {
      const float ea = __expf(lo - m), eb = __expf(lse - m);
      const float sum = ea + eb;
      wa = ea / sum; wb = eb / sum;
      lse_out = m + logf(sum);
    }
  }
  float sink_f = 1.f;
  if (p.sinks) {
    const float sk = p.sinks[qh];
    sink_f = (lse_out == -INFINITY) ? 0.f : 1.f / (1.f + __expf(sk - lse_out));
  }
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      bf16_t* dst = orow + 32 * mt + 8 * q4 + 4 * hh;
      float v0 = o[mt][4 * q4] * inv * wb, v1 = o[mt][4 * q4 + 1] * inv * wb;
      float v2 = o[mt][4 * q4 + 2] * inv * wb, v3 = o[mt][4 * q4 + 3] * inv * wb;
      if (w.mode == MODE_INPLACE && wa != 0.f) {
        const u32x2 old = *(const u32x2*)dst;
        v0 += wa * bf16_lo(old[0]); v1 += wa * bf16_hi(old[0]);
        v2 += wa * bf16_lo(old[1]); v3 += wa * bf16_hi(old[1]);
      }
      *(u32x2*)dst = (u32x2){pack_bf16x2(v0 * sink_f, v1 * sink_f), pack_bf16x2(v2 * sink_f, v3 * sink_f)};
    }
  if (lrow && hh == 0) *lrow = p.lse_base2 ? lse_out * kLog2e : lse_out;
}

// ---------------------------------------------------------------------------
// Split-KV merge: rows of one tile group, ROWS rows, nslots partials each.
// Thread layout: D/4 threads per row (4 head dims each).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void merge_kernel(const AttnParams p, int rows_per_tile, int row_blocks) {
  constexpr int TPR = D / 4;      // threads per row
  constexpr int RPB = 256 / TPR;  // rows per block
  const int item_idx = blockIdx.x / row_blocks;
  const int rb = blockIdx.x % row_blocks;
  MergeItem mi;
  if (p.merge) {
    mi = p.merge[item_idx];
  } else {
    const int Q = p.imp.qtiles;
    mi.qtile = item_idx % Q;
    const int rest = item_idx / Q;
    mi.kvh = rest % p.num_kv_heads;
    mi.req = rest / p.num_kv_heads;
    mi.slot_begin = item_idx * p.imp.splits;
    mi.nslots = p.imp.splits;
    mi.mode = p.imp.single_mode;
  }
  const int lr = rb * RPB + threadIdx.x / TPR;
  const int d0 = (threadIdx.x % TPR) * 4;
  if (lr >= rows_per_tile) return;
  const int g = p.group;
  const int q0 = p.qo_indptr ? p.qo_indptr[mi.req] : 0;
  const int nq = p.qo_indptr ? p.qo_indptr[mi.req + 1] - q0 : p.imp.qo_len;
  const int row = mi.qtile * rows_per_tile + lr;
  if (row >= nq * g) return;
  const int n = row / g, j = row - n * g;
  const int qh = mi.kvh * g + j;

  float m = -INFINITY;
  for (int s = 0; s < mi.nslots; ++s)
    m = fmaxf(m, p.part_lse[(long long)(mi.slot_begin + s) * rows_per_tile + lr]);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (m != -INFINITY) {
    for (int s = 0; s < mi.nslots; ++s) {
      const long long prow = (long long)(mi.slot_begin + s) * rows_per_tile + lr;
      const float ls = p.part_lse[prow];
      const float wgt = __expf(ls - m);  // 0 for an empty split (-inf)
      if (wgt > 0.f) {
        const f32x4 v = *(const f32x4*)(p.part_o + prow * D + d0);
        acc += wgt * v;
        wsum += wgt;
      }
    }
  }
  float lse = (wsum > 0.f) ? m + logf(wsum) : -INFINITY;
  const float inv = (wsum > 0.f) ? 1.f / wsum : 0.f;
  acc *= inv;

  bf16_t* dst = (bf16_t*)p.o + (long long)mi.req * p.o_stride_req + (long long)(q0 + n) * p.o_stride_n +
                (long long)qh * p.o_stride_h + d0;
  float* lrow = p.lse ? p.lse + (long long)mi.req * p.lse_stride_req + (long long)(q0 + n) * p.lse_stride_n + qh
                      : nullptr;
  if (mi.mode == MODE_INPLACE) {
    const float lo = load_lse_nat(lrow, p.lse_base2);
    const float mm = fmaxf(lo, lse);
    if (mm != -INFINITY) {
      const float ea = __expf(lo - mm), eb = __expf(lse - mm);
      const float sum = ea + eb;
      const u32x2 old = *(const u32x2*)dst;
      const f32x4 ov = {bf16_lo(old[0]), bf16_hi(old[0]), bf16_lo(old[1]), bf16_hi(old[1])};
      acc = (ea / sum) * ov + (eb / sum) * acc;
      lse = mm + logf(sum);
    } else {
      const u32x2 old = *(const u32x2*)dst;
      acc = (f32x4){bf16_lo(old[0]), bf16_hi(old[0]), bf16_lo(old[1]), bf16_hi(old[1])};
      lse = -INFINITY;
    }
  }
  if (p.sinks) {
    const float sk = p.sinks[qh];
    acc *= (lse == -INFINITY) ? 0.f : 1.f / (1.f + __expf(sk - lse));
  }
  // all TPR threads of a row have read the stored lse above (same wave)
  *(u32x2*)dst = (u32x2){pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
  if (lrow && d0 == 0) *lrow = p.lse_base2 ? lse * kLog2e : lse;
}

// ---------------------------------------------------------------------------
// merge_state_in_place: one thread per (token, head, 8 head dims).
// ---------------------------------------------------------------------------
struct MergeStateArgs {
  bf16_t* v;
  long long v_sn, v_sh;
  float* s;
  long long s_sn;
  const bf16_t* vo;
  long long vo_sn, vo_sh;
  const float* so;
  long long so_sn;
  int n, h, d, base2;
};

__global__ __launch_bounds__(256) void merge_state_kernel(const MergeStateArgs a) {
  const int chunks = a.d / 8;
  const long long total = (long long)a.n * a.h * chunks;
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    const int c = (int)(i % chunks);
    const long long nh = i / chunks;
    const int h = (int)(nh % a.h);
    const int n = (int)(nh / a.h);
    float* sp = a.s + n * a.s_sn + h;
    const float s1 = a.base2 ? *sp * kLn2 : *sp;
    const float s2 = a.base2 ? a.so[n * a.so_sn + h] * kLn2 : a.so[n * a.so_sn + h];
    const float m = fmaxf(s1, s2);
    bf16_t* vp = a.v + n * a.v_sn + h * a.v_sh + 8 * c;
    const bf16_t* vop = a.vo + n * a.vo_sn + h * a.vo_sh + 8 * c;
    if (m == -INFINITY) continue;  // both empty: state unchanged
    const float e1 = __expf(s1 - m), e2 = __expf(s2 - m);
    const float sum = e1 + e2;
    const float w1 = e1 / sum, w2 = e2 / sum;
    const u32x4 x = *(const u32x4*)vp;
    const u32x4 y = *(const u32x4*)vop;
    u32x4 r;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      r[k] = pack_bf16x2(w1 * bf16_lo(x[k]) + w2 * bf16_lo(y[k]), w1 * bf16_hi(x[k]) + w2 * bf16_hi(y[k]));
    // every chunk thread of (n, h) must read s before one of them writes it:
    // they are consecutive lanes of one wave, which load before they store.
    *(u32x4*)vp = r;
    if (c == 0) {
      const float so = m + logf(sum);
      *sp = a.base2 ? so * kLog2e : so;
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int D, int W, bool FP8>
static hipError_t launch_attn_t(const AttnParams& p, int nblocks, hipStream_t s) {
  hipLaunchKernelGGL((attn_kernel<D, W, FP8>), dim3(nblocks), dim3(64 * W), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnParams& p, int head_dim, int waves, bool fp8, int nblocks,
                            hipStream_t s) {
  if (nblocks <= 0) return hipSuccess;
  if (head_dim == 128) {
    if (waves == 4) return fp8 ? launch_attn_t<128, 4, true>(p, nblocks, s) : launch_attn_t<128, 4, false>(p, nblocks, s);
    if (waves == 8) return fp8 ? launch_attn_t<128, 8, true>(p, nblocks, s) : launch_attn_t<128, 8, false>(p, nblocks, s);
  } else if (head_dim == 64) {
    if (waves == 4) return fp8 ? launch_attn_t<64, 4, true>(p, nblocks, s) : launch_attn_t<64, 4, false>(p, nblocks, s);
    if (waves == 8) return fp8 ? launch_attn_t<64, 8, true>(p, nblocks, s) : launch_attn_t<64, 8, false>(p, nblocks, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_merge(const AttnParams& p, int head_dim, int rows_per_tile, int nitems, hipStream_t s) {
  if (nitems <= 0) return hipSuccess;
  const int tpr = head_dim / 4;
  const int rpb = 256 / tpr;
  const int row_blocks = (rows_per_tile + rpb - 1) / rpb;
  if (head_dim == 128)
    hipLaunchKernelGGL(merge_kernel<128>, dim3(nitems * row_blocks), dim3(256), 0, s, p, rows_per_tile, row_blocks);
  else if (head_dim == 64)
    hipLaunchKernelGGL(merge_kernel<64>, dim3(nitems * row_blocks), dim3(256), 0, s, p, rows_per_tile, row_blocks);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_merge_state(void* v, long long v_sn, long long v_sh, float* s, long long s_sn,
                              const void* vo, long long vo_sn, long long vo_sh, const float* so,
                              long long so_sn, int n, int h, int d, int base2, hipStream_t stream) {
  MergeStateArgs a{(bf16_t*)v, v_sn, v_sh, s, s_sn, (const bf16_t*)vo, vo_sn, vo_sh, so, so_sn, n, h, d, base2};
  const long long total = (long long)n * h * (d / 8);
  if (total == 0) return hipSuccess;
  long long blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(merge_state_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace d2sd
