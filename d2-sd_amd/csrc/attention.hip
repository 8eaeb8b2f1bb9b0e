// gfx950 (CDNA4) kernels of the single-call drop-ins for the reference's
// FlashInfer calls (the cascade plan()/run() path lives in verify_attention.hip):
//
//   attn_dma_kernel     GQA-packed split-KV attention of packed (token, query
//                       head) rows over one contiguous K/V source, unmasked or
//                       causal, with a partial / final / in-place-merge
//                       epilogue.  Replaces flashinfer.single_prefill_with_kv_cache
//                       (generation/verification.py:145-162,
//                       model/cascade_graph.py:54-57) and, with the in-place
//                       epilogue, the per-row local attention + merge loop of
//                       model/cascade_graph.py:52-60.
//   merge_kernel        log-sum-exp merge of split partials (+ the GPT-OSS sink
//                       rescale of generation/verification.py:173-176).
//   merge_state_kernel  flashinfer.merge_state_in_place
//                       (generation/verification.py:163-165, model/cascade_graph.py:58-60).
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
// O^T += V^T . P^T straight from those registers; V^T is read from the
// row-major V tile with ds_read_b64_tr_b16 in the key order of the P^T
// registers.
//
// Register image.  Lane l of wave w holds O^T[d][row] for row = 32w + l%32
// and d = 32*mt + 8*q4 + 4*(l/32) + e (mt < D/32, q4 < 4, e < 4).  Split
// partials (normalised O in bf16, LSE in fp32) are stored in exactly this
// image — the 8 values (mt, q4 = 2pr, 2pr + 1) of lane l at element
// ((w*(D/32) + mt)*2 + pr)*512 + 8*l of the slot — so that every partial
// store and every merge load is one contiguous 1 KB wave access.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "d2sd_internal.h"
#include "kernel_common.h"

namespace d2sd {

__device__ __forceinline__ float load_lse_nat(const float* lse, int base2) {
  const float v = *lse;
  return base2 ? v * kLn2 : v;
}

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

// ---------------------------------------------------------------------------
// Output store of one lane's part of a row (register image), with the
// GPT-OSS sink factor sigmoid(lse - sink); o_scale normalises the values.
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ void store_row(const AttnParams& p, int req, int q0, int n, int qh, int hh,
                                          const f32x16 (&o)[D / 32], float o_scale, float lse) {
  bf16_t* orow = (bf16_t*)p.o + (long long)req * p.o_stride_req + (long long)(q0 + n) * p.o_stride_n +
                 (long long)qh * p.o_stride_h;
  float* lrow = p.lse ? p.lse + (long long)req * p.lse_stride_req + (long long)(q0 + n) * p.lse_stride_n + qh
                      : nullptr;
  if (p.sinks) {
    const float sk = p.sinks[qh];
    o_scale *= (lse == -INFINITY) ? 0.f : 1.f / (1.f + __expf(sk - lse));
  }
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      bf16_t* dst = orow + 32 * mt + 8 * q4 + 4 * hh;
      *(u32x2*)dst = (u32x2){pack_bf16x2(o[mt][4 * q4] * o_scale, o[mt][4 * q4 + 1] * o_scale),
                             pack_bf16x2(o[mt][4 * q4 + 2] * o_scale, o[mt][4 * q4 + 3] * o_scale)};
    }
  if (lrow && hh == 0) *lrow = p.lse_base2 ? lse * kLog2e : lse;
}

// Epilogue of the attention kernel: normalise the accumulators and write a
// split partial or the final output, or merge with the stored state first.
template <int D, int W>
__device__ __forceinline__ void finish_rows(const AttnParams& p, const WorkItem& w, f32x16 (&o)[D / 32],
                                            float m_run, float l_run, float vscale, float cn, int row,
                                            bool rvalid, int q0, int n, int qh) {
  constexpr int ROWS = 32 * W;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, l32 = lane & 31, hh = lane >> 5;
  const int mode = w.mode & 0xff;
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const bool nonempty = l_tot > 0.f;
  const float inv = nonempty ? vscale / l_tot : 0.f;
  float lse = nonempty ? m_run * cn + logf(l_tot) : -INFINITY;
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mt][r] *= inv;

  if (mode == MODE_PARTIAL) {
    bf16_t* po = (bf16_t*)p.part_o + (long long)w.slot * ROWS * D;
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) *(u32x4*)(po + image_offset<D>(wv, mt, pr, lane)) = image_piece(o[mt], pr, 1.f);
    if (hh == 0) p.part_lse[(long long)w.slot * ROWS + wv * 32 + l32] = lse;
    return;
  }
  if (!rvalid) return;

  if (mode == MODE_INPLACE) {
    // merge with the (bf16 O, LSE) state stored at the output
    const bf16_t* orow = (const bf16_t*)p.o + (long long)w.req * p.o_stride_req +
                         (long long)(q0 + n) * p.o_stride_n + (long long)qh * p.o_stride_h;
    const float* lrow = p.lse + (long long)w.req * p.lse_stride_req + (long long)(q0 + n) * p.lse_stride_n + qh;
    const float lo = load_lse_nat(lrow, p.lse_base2);
    const float m = fmaxf(lo, lse);
    float wa = 1.f, wb = 0.f;  // both empty: keep the stored state
    if (m != -INFINITY) {
      const float ea = __expf(lo - m), eb = __expf(lse - m);
      const float sum = ea + eb;
      wa = ea / sum;
      wb = eb / sum;
      lse = m + logf(sum);
    } else {
      lse = lo;
    }
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const u32x2 old = *(const u32x2*)(orow + 32 * mt + 8 * q4 + 4 * hh);
        o[mt][4 * q4] = o[mt][4 * q4] * wb + wa * bf16_lo(old[0]);
        o[mt][4 * q4 + 1] = o[mt][4 * q4 + 1] * wb + wa * bf16_hi(old[0]);
        o[mt][4 * q4 + 2] = o[mt][4 * q4 + 2] * wb + wa * bf16_lo(old[1]);
        o[mt][4 * q4 + 3] = o[mt][4 * q4 + 3] * wb + wa * bf16_hi(old[1]);
      }
  }
  store_row<D>(p, w.req, q0, n, qh, hh, o, 1.f, lse);
}

// ---------------------------------------------------------------------------
// bf16 attention with direct global->LDS tile loads (gfx950).
//
// K and V tiles travel global -> LDS with global_load_lds_dwordx4 (each wave
// instruction writes 1 KB: lane l's 16 bytes at +16*l), into a ring of
// kStages tiles, so up to kStages-1 tiles are in flight per workgroup without
// holding any of them in registers.  Both tiles are stored row-major with the
// 16-byte chunk c of key row r at chunk c ^ swz(r), which makes the K reads
// of the QK MFMA conflict-free.  V is read straight from that row-major tile
// as the A operand of O^T += V^T P^T with ds_read_b64_tr_b16: in every 16-lane
// group lane k names 4 bf16 of key row k/4 and receives column k of the 4 keys,
// so two reads give a lane the 8 keys of its half of a 16-key MFMA step in the
// same order the P^T registers hold them.
// ---------------------------------------------------------------------------
constexpr int kStages = 4;

template <int D>
struct DmaSmem {
  bf16_t ring[kStages][2][64 * D];  // [stage][K, V][key row * D]
  int pages[kMaxStagedPages];
};

template <int D, int W, bool PAGED, bool MASKED>
__device__ __forceinline__ void attn_dma_body(const AttnParams& p, const WorkItem& w, const KvSource& S,
                                              DmaSmem<D>& sm) {
  constexpr int ROWS = 32 * W;
  constexpr int NT = 64 * W;
  constexpr int CH = D / 8;                 // 16-byte chunks per key row
  constexpr int RPI = 64 / CH;              // key rows per 1 KB wave instruction
  constexpr int IPT = 64 / RPI;             // instructions per 64-key tile (K or V)
  constexpr int IPW = IPT / W;              // ... per wave
  constexpr int LPT = 2 * IPW;              // DMA loads per tile per wave (K + V)
  static_assert(IPW >= 1 && IPT % W == 0, "tile/wave mismatch");
  (void)ROWS;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  const int g = p.group;
  const int q0 = p.qo_indptr ? p.qo_indptr[w.req] : 0;
  const int nq = p.qo_indptr ? p.qo_indptr[w.req + 1] - q0 : p.imp.qo_len;
  const int R = nq * g;
  const int row = w.qtile * (32 * W) + wv * 32 + l32;
  const bool rvalid = row < R;
  const int n = rvalid ? row / g : 0;
  const int j = rvalid ? row - n * g : 0;
  const int qh = w.kvh * g + j;

  const float c = p.sm_scale_log2;
  const float cn = p.sm_scale;
  const int kv_begin = w.kv_begin, kv_end = w.kv_end;
  const int ntiles = (kv_end - kv_begin + 63) >> 6;

  int mask_mode = MASK_NONE, causal_off = 0;
  unsigned long long mreg[kMaskRegWords] = {};
  const unsigned long long* mrow = nullptr;
  if constexpr (MASKED) {
    mask_mode = S.mask_mode;
    const int kvlen_req = S.kv_len ? S.kv_len[w.req] : p.imp.kv_len;
    causal_off = kvlen_req - nq;
    if (mask_mode == MASK_TREE && rvalid) {
      mrow = S.tree_mask + (long long)(q0 + n) * S.mask_words;
#pragma unroll
      for (int k = 0; k < kMaskRegWords; ++k) mreg[k] = (k < S.mask_words) ? mrow[k] : 0ull;
    }
  }

  // ---- source addressing (bytes; the kv head is folded into the bases) ----
  const char* kbase = (const char*)S.k + (long long)w.kvh * S.stride_head * 2;
  const char* vbase = (const char*)S.v + (long long)w.kvh * S.stride_head * 2;
  const long long tok_b = S.stride_tok * 2;
  const long long page_b = S.stride_page * 2;
  const int log2p = S.log2_page;
  const int pmask = (1 << log2p) - 1;
  int pg_first = 0;
  if constexpr (PAGED) {
    if (ntiles > 0) {
      pg_first = kv_begin >> log2p;
      const int npg = ((kv_end - 1) >> log2p) - pg_first + 1;  // <= kMaxStagedPages (planner)
      const int* pt = S.page_table + S.page_indptr[w.req] + pg_first;
      for (int i = tid; i < npg; i += NT) sm.pages[i] = pt[i];
    }
  } else {
    const long long base_tok = S.tok_indptr ? S.tok_indptr[w.req] : 0;
    const long long off = ((long long)w.req * S.stride_req + base_tok * S.stride_tok) * 2;
    kbase += off;
    vbase += off;
  }

  // Q fragments (B operand of S^T = K Q^T), loaded while the page ids land
  bf16x8 qf[D / 16];
  {
    const bf16_t* qp = (const bf16_t*)p.q + (long long)w.req * p.q_stride_req +
                       (long long)(q0 + n) * p.q_stride_n + (long long)qh * p.q_stride_h + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
      qf[ks] = rvalid ? *(const bf16x8*)(qp + 16 * ks) : zero_bf16x8();
  }
  // Complete the Q loads here, visibly to the compiler: otherwise it keeps
  // them pending into the tile loop and waits vmcnt(0) there every tile,
  // which would also drain the DMA ring.
  wait_vmcnt<0>();
  __syncthreads();  // page ids visible

  auto tok_off = [&](int t) -> long long {
    if constexpr (PAGED)
      return (long long)sm.pages[(t >> log2p) - pg_first] * page_b + (long long)(t & pmask) * tok_b;
    else
      return (long long)t * tok_b;
  };

  // DMA of tile `it` into ring stage it % kStages.  Keys past kv_end load the
  // last valid key (finite data whose scores the tail mask removes).
  auto issue = [&](int it) {
    const int kb = kv_begin + it * 64;
    bf16_t* kst = &sm.ring[it % kStages][0][0];
    bf16_t* vst = &sm.ring[it % kStages][1][0];
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int inst = wv * IPW + i;
      const int r = inst * RPI + lane / CH;           // key row in the tile
      const int cs = lane % CH;                        // stored chunk
      const int cg = cs ^ chunk_swizzle<D>(r);         // global chunk it holds
      const long long off = tok_off(min(kb + r, kv_end - 1)) + cg * 16;
      dma16(kbase + off, lds_address(kst + inst * 512));
      dma16(vbase + off, lds_address(vst + inst * 512));
    }
  };

  f32x16 o[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mt][r] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;

#pragma unroll
  for (int t = 0; t < kStages - 1; ++t)
    if (t < ntiles) issue(t);

  for (int it = 0; it < ntiles; ++it) {
    // tile `it` has landed once at most min(kStages-2, tiles issued after it)
    // tiles of this wave's DMA are still outstanding; then every wave's share
    // is visible after the barrier, and stage (it-1) % kStages is free.
    const int ahead = min(kStages - 2, ntiles - 1 - it);
    __asm__ volatile("" ::: "memory");  // no LDS access crosses the barrier
    if (ahead >= 2) wait_vmcnt<2 * LPT>();
    else if (ahead == 1) wait_vmcnt<LPT>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    if (it + kStages - 1 < ntiles) issue(it + kStages - 1);

    const int kb = kv_begin + it * 64;
    const bf16_t* kst = &sm.ring[it % kStages][0][0];
    const bf16_t* vst = &sm.ring[it % kStages][1][0];

    // ---- S^T = K Q^T : two 32-key tiles ----
    f32x16 s0, s1;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s0[r] = 0.f; s1[r] = 0.f; }
    {
      const int sw0 = chunk_swizzle<D>(l32), sw1 = chunk_swizzle<D>(l32 + 32);
      const bf16_t* k0 = kst + l32 * D;
      const bf16_t* k1 = kst + (l32 + 32) * D;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const int cidx = 2 * ks + hh;
        const bf16x8 a0 = *(const bf16x8*)(k0 + 8 * (cidx ^ sw0));
        const bf16x8 a1 = *(const bf16x8*)(k1 + 8 * (cidx ^ sw1));
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[ks], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[ks], s1, 0, 0, 0);
      }
    }

    // ---- masking: register r of 32-key tile kt holds key 32*kt + 8*(r/4) + 4*hh + r%4 ----
    bool apply = kb + 64 > kv_end;
    if constexpr (MASKED) apply = apply || mask_mode != MASK_NONE;
    if (apply) {
      unsigned long long mw = ~0ull;
      if constexpr (MASKED) {
        if (mask_mode == MASK_TREE) {
          const int wi = kb >> 6;
          mw = (wi >= kMaskRegWords && mrow) ? mrow[wi] : 0ull;
#pragma unroll
          for (int k = 0; k < kMaskRegWords; ++k) mw = (wi == k) ? mreg[k] : mw;
          if (!rvalid) mw = 0ull;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk0 = 8 * (r >> 2) + 4 * hh + (r & 3);
        const int kk1 = kk0 + 32;
        bool v0 = kb + kk0 < kv_end, v1 = kb + kk1 < kv_end;
        if constexpr (MASKED) {
          if (mask_mode == MASK_CAUSAL) {
            v0 = v0 && (kb + kk0 <= n + causal_off);
            v1 = v1 && (kb + kk1 <= n + causal_off);
          } else if (mask_mode == MASK_TREE) {
            v0 = v0 && ((mw >> kk0) & 1ull);
            v1 = v1 && ((mw >> kk1) & 1ull);
          }
        }
        s0[r] = v0 ? s0[r] : -INFINITY;
        s1[r] = v1 ? s1[r] : -INFINITY;
      }
    }

    // ---- online softmax ----
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

    // ---- O^T += V^T P^T (A operand by transposing LDS reads) ----
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
      // lane k of 16-lane group G names key row 4*hh + k/4 (+8 for the second
      // read) and head dims 16*(G&1) + 4*(k&3) .. +3 of the 32-wide block mt
      const int k16 = lane & 15;
      const int krow = 4 * hh + (k16 >> 2);
      const int dsub = 16 * ((lane >> 4) & 1) + 4 * (k16 & 3);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int key0 = 16 * ks + krow, key1 = key0 + 8;
          const int d = 32 * mt + dsub;
          const bf16_t* p0 = vst + key0 * D + 8 * ((d >> 3) ^ chunk_swizzle<D>(key0)) + (d & 7);
          const bf16_t* p1 = vst + key1 * D + 8 * ((d >> 3) ^ chunk_swizzle<D>(key1)) + (d & 7);
          typedef short s16x4 __attribute__((ext_vector_type(4)));
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p0);
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p1);
          const u32x2 ulo = __builtin_bit_cast(u32x2, lo), uhi = __builtin_bit_cast(u32x2, hi);
          const bf16x8 a = __builtin_bit_cast(bf16x8, (u32x4){ulo[0], ulo[1], uhi[0], uhi[1]});
          o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ks], o[mt], 0, 0, 0);
        }
    }
  }

  finish_rows<D, W>(p, w, o, m_run, l_run, 1.f, cn, row, rvalid, q0, n, qh);
}

template <int D, int W, bool PAGED, bool MASKED, int SRC>
__global__ __launch_bounds__(64 * W) void attn_dma_kernel(const AttnParams p) {
  __shared__ __attribute__((aligned(16))) DmaSmem<D> sm;
  const WorkItem w = implicit_work(p, blockIdx.x);
  if ((w.mode & 0xff) == MODE_NOOP) return;
  attn_dma_body<D, W, PAGED, MASKED>(p, w, p.src[SRC], sm);
}

// ---------------------------------------------------------------------------
// Split-KV merge (single_prefill): one single-wave workgroup per (tile group,
// 32-row block, 32-wide head-dim block mt), so that the partial loads spread
// over every CU; the partials are read in their register image, a batch of
// kMergeBatch slots in flight at once, and the output written like the
// attention kernel's FINAL epilogue (+ the GPT-OSS sink factor).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64) void merge_kernel(const AttnParams p, int rows_per_tile) {
  constexpr int kMergeBatch = 8;
  const int waves_per_tile = rows_per_tile / 32;
  const int item_idx = blockIdx.x / waves_per_tile, blk = blockIdx.x % waves_per_tile, mt = blockIdx.y;
  if (item_idx >= p.num_merge) return;
  const int lane = threadIdx.x, l32 = lane & 31, hh = lane >> 5;
  const int Q = p.imp.qtiles;
  const int qt = item_idx % Q;
  const int rest = item_idx / Q;
  const int kvh = rest % p.num_kv_heads;
  const int req = rest / p.num_kv_heads;
  const int g = p.group;
  const int row = qt * rows_per_tile + blk * 32 + l32;
  if (row >= p.imp.qo_len * g) return;
  const int n = row / g, qh = kvh * g + (row - n * g);
  const int nslots = p.imp.splits;
  const long long slot0 = (long long)item_idx * nslots;
  const long long slot_elems = (long long)rows_per_tile * D;

  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  float mval = -INFINITY, wsum = 0.f;
  for (int s0 = 0; s0 < nslots; s0 += kMergeBatch) {
    float ls[kMergeBatch];
    u32x4 v[kMergeBatch][2];
#pragma unroll
    for (int b = 0; b < kMergeBatch; ++b) {
      ls[b] = -INFINITY;
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) v[b][pr] = (u32x4){0u, 0u, 0u, 0u};
      if (s0 + b < nslots) {
        const long long s = slot0 + s0 + b;
        ls[b] = p.part_lse[s * rows_per_tile + blk * 32 + l32];
        const bf16_t* po = (const bf16_t*)p.part_o + s * slot_elems;
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) v[b][pr] = *(const u32x4*)(po + image_offset<D>(blk, mt, pr, lane));
      }
    }
    float bm = -INFINITY;
#pragma unroll
    for (int b = 0; b < kMergeBatch; ++b) bm = fmaxf(bm, ls[b]);
    const float nm = fmaxf(mval, bm);
    if (nm == -INFINITY) continue;  // nothing visible so far
    const float f = (mval == -INFINITY) ? 0.f : __expf(mval - nm);
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] *= f;
    wsum *= f;
#pragma unroll
    for (int b = 0; b < kMergeBatch; ++b) {
      const float wt = (ls[b] == -INFINITY) ? 0.f : __expf(ls[b] - nm);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[2 * e] += wt * bf16_lo(v[b][e >> 2][e & 3]);
        acc[2 * e + 1] += wt * bf16_hi(v[b][e >> 2][e & 3]);
      }
      wsum += wt;
    }
    mval = nm;
  }
  const bool nonempty = wsum > 0.f;
  const float lse = nonempty ? mval + logf(wsum) : -INFINITY;
  float sc = nonempty ? 1.f / wsum : 0.f;
  if (p.sinks) sc *= nonempty ? 1.f / (1.f + __expf(p.sinks[qh] - lse)) : 0.f;
  bf16_t* orow = (bf16_t*)p.o + (long long)req * p.o_stride_req + (long long)n * p.o_stride_n +
                 (long long)qh * p.o_stride_h;
  store_row_block32(orow + 32 * mt, acc, sc, hh);
  if (p.lse && mt == 0 && hh == 0) {
    float* lrow = p.lse + (long long)req * p.lse_stride_req + (long long)n * p.lse_stride_n + qh;
    *lrow = p.lse_base2 ? lse * kLog2e : lse;
  }
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
template <int D, int W, bool MASKED>
static hipError_t launch_dma_t(const AttnParams& p, int nblocks, hipStream_t s) {
  hipLaunchKernelGGL((attn_dma_kernel<D, W, false, MASKED, 0>), dim3(nblocks), dim3(64 * W), 0, s, p);
  return hipGetLastError();
}

// Kernel variants of the single-source drop-ins: contiguous bf16 K/V,
// unmasked or causal, 4- or 8-wave workgroups.
template <int D>
static hipError_t launch_attention_d(const AttnParams& p, int waves, int src, bool fp8, bool paged, bool masked,
                                     int nblocks, hipStream_t s) {
  if (src != 0 || fp8 || paged) return hipErrorInvalidValue;
  if (waves == 4) return masked ? launch_dma_t<D, 4, true>(p, nblocks, s) : launch_dma_t<D, 4, false>(p, nblocks, s);
  if (waves == 8) return masked ? launch_dma_t<D, 8, true>(p, nblocks, s) : launch_dma_t<D, 8, false>(p, nblocks, s);
  return hipErrorInvalidValue;
}

hipError_t launch_attention(const AttnParams& p, int head_dim, int waves, int src, bool fp8, bool paged,
                            bool masked, int nblocks, hipStream_t s) {
  if (nblocks <= 0) return hipSuccess;
  if (head_dim == 128) return launch_attention_d<128>(p, waves, src, fp8, paged, masked, nblocks, s);
  if (head_dim == 64) return launch_attention_d<64>(p, waves, src, fp8, paged, masked, nblocks, s);
  return hipErrorInvalidValue;
}

hipError_t launch_merge(const AttnParams& p, int head_dim, int rows_per_tile, int nitems, hipStream_t s) {
  if (nitems <= 0) return hipSuccess;
  AttnParams q = p;
  q.num_merge = nitems;
  const dim3 grid((unsigned)(nitems * (rows_per_tile / 32)), (unsigned)(head_dim / 32));
  if (head_dim == 128)
    hipLaunchKernelGGL(merge_kernel<128>, grid, dim3(64), 0, s, q, rows_per_tile);
  else if (head_dim == 64)
    hipLaunchKernelGGL(merge_kernel<64>, grid, dim3(64), 0, s, q, rows_per_tile);
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
