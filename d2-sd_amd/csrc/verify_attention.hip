// gfx950 (CDNA4) kernels of the cascade verify attention plan()/run() path:
//
//   verify_attn_kernel   one launch for both levels of
//                        generation/verification.py:127-165 — workgroups
//                        owning a key chunk of the shared prefix (split-KV,
//                        contiguous or paged, bf16 or fp8 e4m3fn) and
//                        workgroups owning the whole tree-masked suffix.
//                        Each writes a normalised partial state (bf16 O in
//                        its register image + fp32 LSE), or the final output
//                        when it is its group's only producer.
//   verify_merge_kernel  log-sum-exp merge of a group's partials
//                        (flashinfer.merge_state_in_place semantics,
//                        verification.py:163-165) and the GPT-OSS sink rescale
//                        (verification.py:173-176), writing O and LSE.
//
// Rows.  The rows of one (request, kv head) are the packed (query n, query
// head j) pairs, row = n*g + j (g = Hq / Hkv), so all query heads sharing a kv
// head read each key/value element once per workgroup.  A workgroup owns
// ROWS consecutive rows as 32-row MFMA blocks: either two waves of two blocks
// (every K / V^T fragment read from LDS feeds two MFMAs; one wave per SIMD)
// or four / eight waves of one block (two waves per SIMD, so that one wave's
// softmax overlaps the other's MFMAs).
//
// Per 64-key tile a wave computes S^T = K . Q^T (A = K from LDS, B = its Q
// rows held in registers for the whole loop): lane l holds the scores of query
// row l%32 of each block for 32 keys, so softmax max / sum are in-lane plus one
// exchange with lane l^32.  P^T is fed back as the B operand of
// O^T += V^T . P^T straight from registers; the V^T A operand is read with
// ds_read_b64_tr_b16 from the row-major V tile in the key order the P^T
// registers hold.
//
// Key tiles reach LDS by global_load_lds_dwordx4 (bf16 sources) into separate
// K and V rings (K tiles issued one step further ahead than V, since S = K.Q^T
// comes first in a tile), or, for an fp8 prefix, through registers where
// e4m3fn is expanded to bf16 (V stored transposed with permuted key slots).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>
#include <vector>

#include "d2sd_internal.h"
#include "kernel_common.h"

namespace d2sd {

// Direct-to-LDS rings of one workgroup: KST K tiles and VST = KST - 1 V tiles
// (64 keys x D, chunk-swizzled rows), so that K tiles are issued two steps
// ahead and V tiles one; NPG staged page ids (0: page ids come from scalar
// loads of the page table).  Sized to the LDS share of a workgroup: 160 KB
// per CU, two workgroups per CU for 4-wave tiles, one for 8-wave tiles.
template <int D, int WPB>
struct RingCfg;
template <>
struct RingCfg<128, 1> { static constexpr int KST = 3, VST = 2, NPG = 0; };  // 80 KB
template <>
struct RingCfg<128, 2> { static constexpr int KST = 3, VST = 2, NPG = 0; };  // 80 KB
template <>
struct RingCfg<128, 4> { static constexpr int KST = 3, VST = 2, NPG = 0; };  // 80 KB
template <>
struct RingCfg<128, 8> { static constexpr int KST = 4, VST = 3, NPG = kMaxStagedPages; };  // 116 KB
template <>
struct RingCfg<64, 1> { static constexpr int KST = 5, VST = 4, NPG = kMaxStagedPages; };  // 76 KB
template <>
struct RingCfg<64, 2> { static constexpr int KST = 5, VST = 4, NPG = kMaxStagedPages; };  // 76 KB
template <>
struct RingCfg<64, 4> { static constexpr int KST = 5, VST = 4, NPG = 0; };  // 76 KB (page ids by scalar loads)
template <>
struct RingCfg<64, 8> { static constexpr int KST = 6, VST = 5, NPG = kMaxStagedPages; };  // 92 KB

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wzero-length-array"
template <int D, int KST, int VST, int NPG>
struct VerifySmem {
  union {
    struct {
      bf16_t k[KST][64 * D];           // direct-to-LDS K tiles
      bf16_t v[VST][64 * D];           // direct-to-LDS V tiles
      int pages[NPG];                  // page ids of the workgroup's key range
    } ring;
    struct {
      bf16_t k[2][64 * D];             // register-staged K tiles (layout of the rings)
      bf16_t v[2][64 * D];             // register-staged V tiles (layout of the rings)
      int pages[kMaxStagedPages];
    } st;
  };
};
#pragma clang diagnostic pop

// vmcnt <= k * UNIT for a wave-uniform k in [0, MAXK]
template <int UNIT, int MAXK>
__device__ __forceinline__ void wait_vmcnt_units(int k) {
  static_for<MAXK + 1>([&](auto i) {
    if (k == (int)decltype(i)::value) wait_vmcnt<decltype(i)::value * UNIT>();
  });
}

// Element offset of packed row `row` = (node row / g, head row % g) of a
// group, stepped `step` rows at a time without a division per step; rows
// past the group's end (R rows) give the last row's offset (valid() false).
struct RowWalk {
  int row, j, step, dj, g, R;
  long long off, dstep, wrap, last;
  __device__ __forceinline__ RowWalk(int row0, int step_, int R_, int g_, long long sn, long long sh)
      : row(row0), step(step_), g(g_), R(R_) {
    const int n0 = row0 / g_;
    j = row0 - n0 * g_;
    off = (long long)n0 * sn + (long long)j * sh;
    dj = step_ % g_;
    dstep = (long long)(step_ / g_) * sn + (long long)dj * sh;
    wrap = sn - (long long)g_ * sh;
    const int nl = (R_ - 1) / g_;
    last = (long long)nl * sn + (long long)(R_ - 1 - nl * g_) * sh;
  }
  __device__ __forceinline__ bool valid() const { return row < R; }
  __device__ __forceinline__ long long offset() const { return row < R ? off : last; }
  __device__ __forceinline__ void next() {
    row += step;
    off += dstep;
    j += dj;
    if (j >= g) {
      j -= g;
      off += wrap;
    }
  }
};

// Row value of the partner lane l ^ 32 (the other half of the wave), by
// v_permlane32_swap: after swapping the upper half of `a` with the lower half
// of `b` (both copies of x), lane l < 32 finds x[l + 32] in b and lane l >= 32
// finds x[l - 32] in a.
__device__ __forceinline__ float xor32(float x, int hh) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(hh ? r[0] : r[1]);
}

// Online-softmax state of a wave's RB row blocks: O^T accumulators, the
// running max (raw-score units of the source being read) and this lane's part
// of the row sums, and the rows' Q fragments.
template <int RB, int MT, int KS>
struct VerifyState {
  f32x16 o[RB][MT];
  float m_run[RB], l_run[RB];
  bf16x8 qf[RB][KS];
  // handed from a fused item's prefix level to its suffix level: the suffix's
  // first tiles were issued into the ring rotated by ring_off (handoff != 0)
  // and its rows' tree-mask words loaded
  int handoff, ring_off;
  unsigned long long mreg[RB][kMaskRegWords];
  // dynamic plans: request 0's run-time prefix length, loaded at kernel entry
  // together with the item (the other requests' lengths are loaded after it)
  int len0;
};

// One workgroup: rows [qtile*ROWS, +ROWS) of (req, kvh) against keys
// [kv_begin, kv_end) of source S.  Each of the W waves owns RB 32-row
// blocks (ROWS = 32*RB*W).
//   PAGED  : S is a paged pool (the range's page ids are staged in LDS)
//   MASKED : the suffix level (causal / tree / no mask; else only the
//            key-range tail is masked)
//   FP8    : S holds e4m3fn bytes, staged through registers
//   INIT   : start from an empty state and load the Q fragments; else
//            continue the state of an earlier call (suffix level only)
//   EPI    : normalise and store (partial slot or output); else leave the
//            state for a following suffix-level call, O in value units and
//            the running max in bf16 score units (prefix level only)
//   INPLACE: the items merge into the (O, LSE) already stored at the output
//            (MODE_INPLACE, suffix level only); the stored state is loaded
//            with Q, so its round trip overlaps the first tiles
// SEAM (fused items, bf16 prefix): 1 = the prefix level issues the suffix
// level's first tiles and mask words during its last tile; 2 = the suffix
// level continues from them.
template <int D, int W, int RB, int KST, int VST, int NPG, bool PAGED, bool MASKED, bool FP8, bool INIT = true,
          bool EPI = true, bool INPLACE = false, int SEAM = 0>
__device__ __forceinline__ void verify_body(const VerifyParams& p, const VerifyItem& w, const VerifySource& S,
                                            VerifySmem<D, KST, VST, NPG>& sm,
                                            VerifyState<RB, D / 32, D / 16>& st) {
  static_assert(INIT || MASKED, "only the suffix level continues a state");
  static_assert(EPI || !MASKED, "the suffix level always ends a state");
  static_assert(!INPLACE || (MASKED && INIT && EPI), "in-place merges end a suffix-level state");
  constexpr int ROWS = 32 * RB * W;
  constexpr int NT = 64 * W;
  constexpr int MT = D / 32;
  constexpr int KS = D / 16;
  constexpr int ESZ = FP8 ? 1 : 2;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  const int g = p.group;
  const int R = w.nq * g;
  const int wrow0 = w.qtile * ROWS + wv * 32 * RB;
  const bool live = wrow0 < R;  // wave-uniform: the wave owns at least one valid row
  int n[RB], qh[RB];
  bool rv[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = wrow0 + 32 * rb + l32;
    rv[rb] = row < R;
    n[rb] = rv[rb] ? row / g : 0;
    qh[rb] = w.kvh * g + (rv[rb] ? row - n[rb] * g : 0);
  }
  int kv_begin = w.kv_begin, kv_end = w.kv_end;
  if constexpr (!MASKED) {
    // dynamic plan: the run-time span [k0, L) (L never beyond the planned
    // length) in 64-key tiles from k0, the last one ending at L.  A chunk of
    // the whole span takes its share of the partition the planner made at the
    // planned length (dyn_chunk_start: even shares, the first chunks one tile
    // longer); a chunk of a piece scales its planned boundaries, rounded down
    // to a tile, so the chunks stay contiguous, keep their relative sizes (the
    // plan's balance over XCDs and CUs) and no workgroup idles on keys past L
    if (p.prefix_len || p.prefix_len_set) {
      const int L = min(max(p.prefix_len_set ? p.prefix_len_value : w.req == 0 ? st.len0 : p.prefix_len[w.req], 0),
                        w.plan_len);
      const int span = p.window_left >= 0 ? min(L, p.window_left) : L;
      const int k0 = L - span;
      if (w.chunk) {
        const int c = w.chunk & 0xffff, S = w.chunk >> 16, nt = (span + 63) >> 6;
        kv_begin = k0 + min(span, 64 * dyn_chunk_start(c, S, nt));
        kv_end = k0 + min(span, 64 * dyn_chunk_start(c + 1, S, nt));
      } else {
        const long long pspan = (long long)w.plan_len - w.kv0;
        auto scale = [&](int x) -> int {
          if (pspan <= 0 || x >= pspan) return span;
          return min(span, (int)(((long long)x * span / pspan) & ~63ll));
        };
        kv_begin = k0 + scale(w.kv_begin - w.kv0);
        kv_end = k0 + scale(w.kv_end - w.kv0);
      }
    }
  }
  const int ntiles = kv_end > kv_begin ? (kv_end - kv_begin + 63) >> 6 : 0;

  // ---- suffix masks: the rows' tree-mask words held in registers ----
  int mask_mode = MASK_NONE;
  unsigned long long mreg[RB][kMaskRegWords];
  const unsigned long long* mrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    mrow[rb] = nullptr;
#pragma unroll
    for (int k = 0; k < kMaskRegWords; ++k) mreg[rb][k] = 0ull;
  }
  if constexpr (MASKED) {
    mask_mode = p.mask_mode;
    if (mask_mode == MASK_TREE) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        if (rv[rb]) {
          mrow[rb] = p.tree_mask + (long long)(w.q0 + n[rb]) * p.mask_words;
#pragma unroll
          for (int k = 0; k < kMaskRegWords; ++k)
            mreg[rb][k] = (SEAM == 2 && st.handoff) ? st.mreg[rb][k] : (k < p.mask_words) ? mrow[rb][k] : 0ull;
        }
    }
  }
  auto tile_word = [&](int rb, int wi) -> unsigned long long {
    unsigned long long m = (wi >= kMaskRegWords && mrow[rb]) ? mrow[rb][wi] : 0ull;
#pragma unroll
    for (int k = 0; k < kMaskRegWords; ++k) m = (wi == k) ? mreg[rb][k] : m;
    return m;
  };

  // ---- source addressing (bytes; the kv head is folded into the bases) ----
  const char* kbase = (const char*)S.k + (long long)w.kvh * S.stride_head * ESZ;
  const char* vbase = (const char*)S.v + (long long)w.kvh * S.stride_head * ESZ;
  const long long tok_b = S.stride_tok * ESZ;
  const long long page_b = S.stride_page * ESZ;
  const int log2p = S.log2_page;
  const int pmask = (1 << log2p) - 1;
  // ---- page ids of the key range: loaded first, so that staging them (and
  // issuing the first key tiles) waits for these loads only, not for Q ----
  constexpr int PPT = (kMaxStagedPages + NT - 1) / NT;  // page ids per thread
  // page ids staged in LDS (else read from the page table by scalar loads)
  constexpr bool STAGED = PAGED && (FP8 || NPG > 0);
  int* const pages = FP8 ? sm.st.pages : sm.ring.pages;
  int pg_first = 0, npg = 0;
  int pgv[PPT];
  if constexpr (STAGED) {
    if (ntiles > 0) {
      pg_first = kv_begin >> log2p;
      // the planner keeps every chunk within kMaxStagedPages pages; the clamp
      // only bounds what a bad plan can reach (keys past the staged pages
      // then read the last staged page, never an unstaged LDS word)
      npg = min(((kv_end - 1) >> log2p) - pg_first + 1, kMaxStagedPages);
      const int* pt = S.page_table + w.base + pg_first;
      // unconditional (index clamped into the range) so that the wait before
      // the LDS stores below counts exactly the loads issued after these
#pragma unroll
      for (int j = 0; j < PPT; ++j) pgv[j] = pt[min(tid + j * NT, npg - 1)];
#pragma unroll
      for (int j = 0; j < PPT; ++j) pgv[j] = (int)min((unsigned)pgv[j], (unsigned)S.num_pages - 1u);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- Q fragments (B operand of S^T = K Q^T): lane holds 8 consecutive
  // head dims at offset 8*hh of every 16-wide k step, for row block rb.  The
  // bf16 prefix level stages Q through LDS (below); the others load it here ----
  auto& qf = st.qf;
  auto load_q = [&]() {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const bf16_t* qp = (const bf16_t*)p.q + (long long)(w.q0 + n[rb]) * p.q_stride_n +
                         (long long)qh[rb] * p.q_stride_h + 8 * hh;
#pragma unroll
      // unconditional: rows past the group's end read a valid row (node 0);
      // their results are never stored or merged
      for (int ks = 0; ks < KS; ++ks) qf[rb][ks] = *(const bf16x8*)(qp + 16 * ks);
    }
  };
  if constexpr ((MASKED || FP8) && INIT) load_q();
  // INPLACE: the stored output of this wave's rows, read row by row (lane:
  // 16-byte piece lane % OCH of row ORPI i + lane / OCH of each 32-row block,
  // so that one instruction reads whole rows) and their stored LSE; the
  // epilogue moves the pieces into the MFMA layout through LDS
  constexpr int OCH = D / 8, ORPI = 64 / OCH, OIPB = 32 / ORPI;
  u32x4 old_o[RB][INPLACE ? OIPB : 1];
  float old_lse[RB];
  if constexpr (INPLACE) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      // raw (base-2 when lse_base2): converted in the epilogue, so that no
      // instruction waits for this load before the key tiles are issued
      old_lse[rb] = -INFINITY;
      if (rv[rb]) old_lse[rb] = p.lse[(long long)(w.q0 + n[rb]) * p.lse_stride_n + qh[rb]];
      // unconditional (rows past the group's end read its last row, never
      // stored): a load under a branch would be waited for at the join
      RowWalk rw(wrow0 + 32 * rb + lane / OCH, ORPI, R, g, p.o_stride_n, p.o_stride_h);
      const bf16_t* obase = (const bf16_t*)p.o + (long long)w.q0 * p.o_stride_n +
                            (long long)(w.kvh * g) * p.o_stride_h + 8 * (lane % OCH);
#pragma unroll
      for (int i = 0; i < OIPB; ++i, rw.next()) old_o[rb][i] = *(const u32x4*)(obase + rw.offset());
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (STAGED) {
#pragma unroll
    for (int j = 0; j < PPT; ++j)
      if (tid + j * NT < npg) pages[tid + j * NT] = pgv[j];
  } else if constexpr (PAGED) {
    if (ntiles > 0) pg_first = kv_begin >> log2p;
  } else {
    const long long off = (long long)w.base * tok_b;
    kbase += off;
    vbase += off;
  }

  float kscale = 1.f, vscale = 1.f;
  if constexpr (FP8) {
    // e4m3fn bytes are expanded to their exact values (fp8x4_to_bf16x4)
    kscale = S.k_scale ? S.k_scale[w.kvh] : 1.f;
    vscale = S.v_scale ? S.v_scale[w.kvh] : 1.f;
  }
  const float c = p.sm_scale_log2 * kscale;  // raw score -> log2 domain
  const float cn = p.sm_scale * kscale;      // raw score -> natural domain
  const float slack_raw = c > 0.f ? kRescaleSlack / c : 0.f;  // kRescaleSlack in raw-score units

  // page ids visible (each thread's stores waited for its page-id loads only);
  // nothing to publish when they are not staged
  if constexpr (STAGED) __syncthreads();

  auto tok_off = [&](int t) -> long long {
    if constexpr (STAGED)
      return (long long)pages[min((unsigned)((t >> log2p) - pg_first), (unsigned)max(npg - 1, 0))] * page_b +
             (long long)(t & pmask) * tok_b;
    else if constexpr (PAGED)
      return (long long)min((unsigned)S.page_table[w.base + (t >> log2p)], (unsigned)S.num_pages - 1u) * page_b +
             (long long)(t & pmask) * tok_b;
    else
      return (long long)t * tok_b;
  };

  auto& o = st.o;
  auto& m_run = st.m_run;
  auto& l_run = st.l_run;
  if constexpr (INIT) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[rb][mt][r] = 0.f;
      m_run[rb] = -INFINITY;
      l_run[rb] = 0.f;
    }
  }

  // Whether any row of this wave sees a key of tile kb (suffix masks).
  auto tile_visible = [&](int kb) -> bool {
    if constexpr (MASKED) {
      if (mask_mode == MASK_TREE) {
        unsigned long long any = 0ull;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) any |= tile_word(rb, kb >> 6);
        return __any(any != 0ull);
      }
      if (mask_mode == MASK_CAUSAL) {
        bool any = false;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) any = any || (rv[rb] && kb <= n[rb] + w.causal_off);
        return __any(any);
      }
    }
    return true;
  };

  // Suffix level: some row of this wave sees a key of kb + 32 .. kb + 63
  // (else the in-place kind skips the tile's upper half: past the range, or
  // masked for every row, as for the drop-in runner's blocks of up to 32
  // tokens)
  auto upper_visible = [&](int kb) -> bool {
    if (kv_end - kb <= 32) return false;
    if constexpr (MASKED) {
      if (mask_mode == MASK_TREE) {
        unsigned long long any = 0ull;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) any |= tile_word(rb, kb >> 6);
        return __any((any >> 32) != 0ull);
      }
      if (mask_mode == MASK_CAUSAL) {
        bool any = false;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) any = any || (rv[rb] && kb + 32 <= n[rb] + w.causal_off);
        return __any(any);
      }
    }
    return true;
  };

  // Pieces of one 64-key tile.  kfrag(kt, ks) is the A operand of keys
  // 32kt..32kt+31, head dims 16ks.. (this lane's part); vfrag(mt, ks) the A
  // operand of head dims 32mt.., keys 16ks.. in P^T order.

  // S^T += K Q^T over head dims 16ks..16ks+15 (ks == 0 starts from zero)
  auto qk_ks = [&](f32x16 (&s)[RB][2], auto&& kfrag, int ks) {
    const bf16x8 a0 = kfrag(0, ks);
    const bf16x8 a1 = kfrag(1, ks);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      s[rb][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[rb][ks], ks == 0 ? f32x16{} : s[rb][0], 0, 0, 0);
      s[rb][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[rb][ks], ks == 0 ? f32x16{} : s[rb][1], 0, 0, 0);
    }
  };

  // masking.  vis (bit kk = key kb + kk visible) per row block; register r
  // of 32-key tile kt holds key 32*kt + 8*(r/4) + 4*hh + r%4, i.e. bit
  // 8*(r/4) + r%4 of the row's 32-bit half kt shifted down by 4*hh.
  auto mask_scores = [&](f32x16 (&s)[RB][2], int kb, auto masked_tile) {
    if constexpr (decltype(masked_tile)::value) {
      const int rem = kv_end - kb;  // > 0: tile it < ntiles
      const unsigned long long tail = rem >= 64 ? ~0ull : ((1ull << rem) - 1ull);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        unsigned long long vis = tail;
        if constexpr (MASKED) {
          if (mask_mode == MASK_TREE) {
            vis &= rv[rb] ? tile_word(rb, kb >> 6) : 0ull;
          } else if (mask_mode == MASK_CAUSAL) {
            const int lim = n[rb] + w.causal_off - kb;  // keys kk <= lim are visible
            vis &= lim >= 63 ? ~0ull : (lim < 0 ? 0ull : ((2ull << lim) - 1ull));
          }
        }
        const unsigned lo = (unsigned)vis >> (4 * hh);
        const unsigned hi = (unsigned)(vis >> 32) >> (4 * hh);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int bit = 8 * (r >> 2) + (r & 3);
          s[rb][0][r] = ((lo >> bit) & 1u) ? s[rb][0][r] : -INFINITY;
          s[rb][1][r] = ((hi >> bit) & 1u) ? s[rb][1][r] : -INFINITY;
        }
      }
    }
  };

  // Online softmax (lane-local row, partner lane l^32).  The running max
  // m_run lags the true row max by up to kRescaleSlack (log2 units) before O
  // and l are rescaled, so the rescale branch is rare.  mc = m_run * c is
  // the exponent offset of the tile's probabilities.
  auto max_rescale = [&](const f32x16 (&s)[RB][2], float (&mc)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      // row max: three-input maxima over four independent chains
      float m4[4] = {s[rb][0][0], s[rb][0][1], s[rb][0][2], s[rb][0][3]};
#pragma unroll
      for (int r = 4; r < 16; ++r) m4[r & 3] = fmaxf(m4[r & 3], s[rb][0][r]);
#pragma unroll
      for (int r = 0; r < 16; ++r) m4[r & 3] = fmaxf(m4[r & 3], s[rb][1][r]);
      float mx = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
      mx = fmaxf(mx, xor32(mx, hh));
      // grow iff mx exceeds m_run by more than the slack (always when m_run is
      // -inf and mx finite; never when the row sees nothing yet)
      if (__any(mx > m_run[rb] + slack_raw)) {
        const float m_new = fmaxf(m_run[rb], mx);
        const float alpha = (m_run[rb] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((m_run[rb] - m_new) * c);
        l_run[rb] *= alpha;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) o[rb][mt] *= alpha;
        m_run[rb] = m_new;
      }
      mc[rb] = (m_run[rb] == -INFINITY) ? 0.f : m_run[rb] * c;
    }
  };

  // P^T (bf16) of keys 16j..16j+15 of row block rb.  The row sum adds the
  // fp32 probabilities: a sum of the bf16-rounded P would be off by up to
  // 2^-9 relative for rows that see only a few keys (tree rows near the
  // root), beyond the LSE tolerance.
  auto p_chunk = [&](const f32x16 (&s)[RB][2], int rb, int j, float mc_, float (&ls)[4]) -> bf16x8 {
    const f32x16& sv = s[rb][j >> 1];
    const int base = 8 * (j & 1);
    float pv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pv[i] = __builtin_amdgcn_exp2f(fmaf(sv[base + i], c, -mc_));
      ls[i & 3] += pv[i];
    }
    u32x4 u;
    u[0] = pack_bf16x2(pv[0], pv[1]);
    u[1] = pack_bf16x2(pv[2], pv[3]);
    u[2] = pack_bf16x2(pv[4], pv[5]);
    u[3] = pack_bf16x2(pv[6], pv[7]);
    return __builtin_bit_cast(bf16x8, u);
  };

  // O^T += V^T P^T over keys 16j..16j+15: consecutive MFMAs update
  // different accumulators
  auto pv_chunk = [&](auto&& vfrag, const bf16x8 (&pb)[RB][4], int j) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const bf16x8 a = vfrag(mt, j);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        o[rb][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[rb][j], o[rb][mt], 0, 0, 0);
    }
  };

  // The remaining softmax and PV of a tile whose scores s are final.
  auto finish_tile = [&](const f32x16 (&s)[RB][2], auto&& vfrag) {
    float mc[RB];
    max_rescale(s, mc);
    bf16x8 pb[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float ls[4] = {0.f, 0.f, 0.f, 0.f};  // four independent add chains
#pragma unroll
      for (int j = 0; j < 4; ++j) pb[rb][j] = p_chunk(s, rb, j, mc[rb], ls);
      l_run[rb] += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) pv_chunk(vfrag, pb, j);
  };

  // One whole 64-key tile: QK^T, masking, online softmax, PV.
  auto compute_tile = [&](int kb, auto&& kfrag, auto&& vfrag, auto masked_tile) {
    f32x16 s[RB][2];
    // (the in-place kind only: one wave per SIMD leaves room for the second
    // path; in the split kinds it would spill registers of the prefix loop)
    if constexpr (INPLACE && RB == 1) {
      if (!upper_visible(kb)) {
        // half a tile: QK^T, softmax and PV of keys kb .. kb + 31 only
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8 a0 = kfrag(0, ks);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
            s[rb][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[rb][ks], ks == 0 ? f32x16{} : s[rb][0], 0, 0, 0);
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[rb][1][r] = -INFINITY;
        mask_scores(s, kb, masked_tile);
        float mc[RB];
        max_rescale(s, mc);
        bf16x8 pb[RB][4];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < 2; ++j) pb[rb][j] = p_chunk(s, rb, j, mc[rb], ls);
          l_run[rb] += (ls[0] + ls[1]) + (ls[2] + ls[3]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) pv_chunk(vfrag, pb, j);
        return;
      }
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qk_ks(s, kfrag, ks);
    mask_scores(s, kb, masked_tile);
    finish_tile(s, vfrag);
  };

  // Software-pipelined tile step (unmasked prefix tiles): the softmax and PV
  // of the current tile (scores sc) interleaved with QK^T of the next tile
  // (kfrag_n), which becomes sc.  MFMA and VALU work of one wave then
  // overlap: the QK^T MFMAs are independent of the softmax.  The 16-key P
  // chunk j is converted while PV of chunk j-1 runs.
  auto pipelined_tile = [&](f32x16 (&sc)[RB][2], auto&& kfrag_n, auto&& vfrag) {
    constexpr int Q1 = KS / 4;  // QK^T k-steps beside the row max
    // A wave computing a tile step wins instruction issue over a wave of its
    // SIMD that is at its step's wait and DMA issue (attention launch of a
    // 150-node Qwen3-8B tree over a 4096-key paged prefix -2.3%, of the
    // GPT-OSS-20B head shape over 8192 keys -1.4%, other shapes within noise;
    // A/B in one session).
    __builtin_amdgcn_s_setprio(1);
    f32x16 sn[RB][2];
    static_for<Q1>([&](auto ks) { qk_ks(sn, kfrag_n, decltype(ks)::value); });
    float mc[RB];
    max_rescale(sc, mc);
    float ls[RB][4];
    bf16x8 pb[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) ls[rb][i] = 0.f;
    }
    // QK^T k-steps [Q1 + (j (KS - Q1)) / 4, Q1 + ((j + 1)(KS - Q1)) / 4) go with chunk j
    static_for<4>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) pb[rb][j] = p_chunk(sc, rb, j, mc[rb], ls[rb]);
      if constexpr (j > 0) pv_chunk(vfrag, pb, j - 1);
      constexpr int k0 = Q1 + (j * (KS - Q1)) / 4, k1 = Q1 + ((j + 1) * (KS - Q1)) / 4;
      static_for<k1 - k0>([&](auto kk) { qk_ks(sn, kfrag_n, k0 + decltype(kk)::value); });
    });
    pv_chunk(vfrag, pb, 3);
    // the scheduler's MFMA / LDS-read interleave for this region (measured
    // 0.5% faster at one request of 4096 keys, 3% at eight of 8K-32K)
    __builtin_amdgcn_iglp_opt(0);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      l_run[rb] += (ls[rb][0] + ls[rb][1]) + (ls[rb][2] + ls[rb][3]);
      sc[rb][0] = sn[rb][0];
      sc[rb][1] = sn[rb][1];
    }
    __builtin_amdgcn_s_setprio(0);
  };

  if constexpr (!FP8) {
    // ================= direct global -> LDS rings (bf16 sources) =================
    constexpr int CH = D / 8;      // 16-byte chunks per key row
    constexpr int RPI = 64 / CH;   // key rows per 1 KB wave instruction
    constexpr int IPT = 64 / RPI;  // instructions per 64-key tile (K or V)
    constexpr int IPW = IPT / W;   // ... per wave
    constexpr int TB = 64 * D * 2; // bytes of one K or V tile
    static_assert(IPW >= 1 && IPT % W == 0, "tile/wave mismatch");
    static_assert(KST == VST + 1 && VST >= 2, "ring depths");
    // loads that may still be outstanding when tile `it` has landed (below)
    constexpr int MAXK = 1 + (VST - 2) + (VST - 2);
    static_assert(MAXK * IPW < 64, "vmcnt range");

    const unsigned kring = __builtin_amdgcn_readfirstlane(lds_address(&sm.ring.k[0][0]));
    const unsigned vring = __builtin_amdgcn_readfirstlane(lds_address(&sm.ring.v[0][0]));
    // Per-lane part of the source offset of DMA instruction i: key row
    // lrow of its RPI-row group, stored chunk cs holding global chunk
    // cs ^ swizzle(row).  A wave's instructions cover WROWS consecutive key
    // rows of a tile.  Fast path: full tiles of an item whose key range starts
    // on a 64-key boundary and, paged, whose pages hold 16..64 keys and at
    // least WROWS or 16 of them: each half of the wave's rows then lies in one
    // page at a fixed in-page row (one page for WROWS <= 16, at most two for
    // the 32 rows of a two-wave workgroup), so one wave-uniform base per half
    // and tile (page id * page bytes, a 32 x 32 -> 64-bit scalar multiply)
    // plus this per-lane constant addresses every DMA.
    constexpr int WROWS = IPW * RPI;
    const int lrow = lane / CH, cs = lane % CH;
    const int P = 1 << log2p;
    const bool fast = (kv_begin & 63) == 0 && tok_b < (1ll << 26) &&
                      (!PAGED || (P >= min(WROWS, 16) && P <= 64 && page_b < (1ll << 32)));
    unsigned lane_off[IPW];
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int r0 = (wv * IPW + i) * RPI;  // first row of the instruction in the tile
      const int row_in_src = PAGED ? (r0 & pmask) : r0;
      lane_off[i] = (unsigned)((row_in_src + lrow) * tok_b) + (unsigned)((cs ^ chunk_swizzle<D>(r0 + lrow)) * 16);
    }
    // Page ids of the two halves of this wave's rows of tile `it` (fast path;
    // equal unless WROWS > 16; tiles past the range clamp to its last page),
    // fetched one step before they are needed: from the staged list, or by
    // scalar loads of the page table.
    const int last_page = ntiles > 0 ? (kv_end - 1) >> log2p : 0;
    struct PagePair {
      int a, b;
    };
    auto wave_page = [&](int it) -> PagePair {
      if constexpr (PAGED) {
        auto page_of = [&](int row) -> int {
          const int pi = min(row >> log2p, last_page);
          if constexpr (STAGED) {
            return pages[min(max(pi - pg_first, 0), max(npg - 1, 0))];
          } else {
            typedef const __attribute__((address_space(4))) int const_int;
            return ntiles > 0
                       ? (int)min((unsigned)((const_int*)S.page_table)[w.base + pi], (unsigned)S.num_pages - 1u)
                       : 0;
          }
        };
        const int r = kv_begin + it * 64 + wv * WROWS;
        const int a = page_of(r);
        return {a, WROWS > 16 ? page_of(r + WROWS / 2) : a};
      }
      return {0, 0};
    };

    // DMA of K (or V) of tile `it` into its ring slot.  Keys past kv_end (tail
    // tile only) load the last valid key: finite data whose scores the tail
    // mask removes.
    auto issue = [&](int it, PagePair pg, const char* base, unsigned slot_lds) {
      const int kb = kv_begin + it * 64;
      if (fast && kb + 64 <= kv_end) {
        unsigned long long ua, ub;
        if constexpr (PAGED) {
          ua = (unsigned long long)(unsigned)__builtin_amdgcn_readfirstlane(pg.a) * (unsigned)page_b;
          ub = (unsigned long long)(unsigned)__builtin_amdgcn_readfirstlane(pg.b) * (unsigned)page_b;
        } else {
          ua = ub = (unsigned long long)(unsigned)kb * (unsigned)tok_b;
        }
#pragma unroll
        for (int i = 0; i < IPW; ++i)
          dma16s(base + ((WROWS > 16 && i >= IPW / 2) ? ub : ua), lane_off[i], slot_lds + (wv * IPW + i) * 1024);
      } else {
#pragma unroll
        for (int i = 0; i < IPW; ++i) {
          const int inst = wv * IPW + i;
          const int r = inst * RPI + lrow;
          dma16(base + tok_off(min(kb + r, kv_end - 1)) + (cs ^ chunk_swizzle<D>(r)) * 16, slot_lds + inst * 1024);
        }
      }
    };
    // ring slots: K(it) in (it + roff) % KST, V(it) in (it + roff) % VST
    // (roff != 0 only for a suffix level continuing a fused item's ring)
    int roff = 0;
    if constexpr (SEAM == 2) roff = st.handoff ? st.ring_off : 0;
    auto issue_k = [&](int it, PagePair pg) { issue(it, pg, kbase, kring + ((it + roff) % KST) * TB); };
    auto issue_v = [&](int it, PagePair pg) { issue(it, pg, vbase, vring + ((it + roff) % VST) * TB); };

    // LDS byte offsets (inside a tile) of this lane's fragments; the
    // key-row / head-dim steps are immediate offsets.  K: key row l32 (+32 for
    // kt = 1), chunk (2ks + hh) ^ swizzle.  V^T for ds_read_b64_tr_b16: lane k
    // of a 16-lane group G names key row 4*hh + k/4 (+8 for the second read,
    // +16ks) and head dims 16*(G&1) + 4*(k&3) .. +3 of the 32-wide block mt.
    unsigned koff[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) koff[ks] = (l32 * D + 8 * ((2 * ks + hh) ^ chunk_swizzle<D>(l32))) * 2;
    const int k16 = lane & 15;
    const int krow = 4 * hh + (k16 >> 2);
    const int dsub = 16 * ((lane >> 4) & 1) + 4 * (k16 & 3);
    unsigned voff0[MT], voff1[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int d = 32 * mt + dsub;
      voff0[mt] = (krow * D + 8 * ((d >> 3) ^ chunk_swizzle<D>(krow)) + (d & 7)) * 2;
      voff1[mt] = ((krow + 8) * D + 8 * ((d >> 3) ^ chunk_swizzle<D>(krow + 8)) + (d & 7)) * 2;
    }
    typedef __attribute__((address_space(3))) char lds_char;

    // Fragment readers of the ring slots holding K(it) / V(it).
    auto kfrag_at = [&](int it) {
      const lds_char* kst = (const lds_char*)(uintptr_t)(kring + ((it + roff) % KST) * TB);
      return [&, kst](int kt, int ks) -> bf16x8 {
        return *(const __attribute__((address_space(3))) bf16x8*)(kst + koff[ks] + kt * 32 * D * 2);
      };
    };
    auto vfrag_at = [&](int it) {
      const lds_char* vst = (const lds_char*)(uintptr_t)(vring + ((it + roff) % VST) * TB);
      return [&, vst](int mt, int ks) -> bf16x8 {
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        const lds_char* p0 = vst + voff0[mt] + ks * 16 * D * 2;
        const lds_char* p1 = vst + voff1[mt] + ks * 16 * D * 2;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p1);
        const u32x2 ulo = __builtin_bit_cast(u32x2, lo), uhi = __builtin_bit_cast(u32x2, hi);
        return __builtin_bit_cast(bf16x8, (u32x4){ulo[0], ulo[1], uhi[0], uhi[1]});
      };
    };

    if constexpr (!MASKED) {
      // ---- prefix level: software-pipelined tiles ----
      // K(j) is read one step before V(j) (QK^T of tile j runs under the
      // softmax of tile j-1).  Issue order: K(0), Q, V(0), K(1), K(2), then
      // V / K pairs for steps -(VST - 2) .. -1, then step s issues
      // V(s + VST - 1) and K(s + KST).  Slots: K(j) in j % KST, V(j) in
      // j % VST; step s refills the slots of K(s) (read in step s-1) and
      // V(s-1).
      //
      // Q: each wave's rows are DMA'd into ring slots the first tiles do not
      // use (K slots 2.., then V slots 1..), in the chunk-swizzled K layout,
      // so that the first QK^T waits for Q and K(0) only (a register load of
      // Q would make the compiler drain every outstanding DMA before its
      // first use); the slots are handed back once all waves hold their Q
      // fragments.
      constexpr int QB = RB * 32 * D * 2;  // bytes of one wave's Q rows
      constexpr int NQI = QB / 1024;       // its DMA instructions
      constexpr int FREE1 = (KST - 2) * TB;
      static_assert(W * QB <= FREE1 + (VST - 1) * TB && TB % QB == 0, "Q staging must fit free ring slots");
      const unsigned qdst = wv * QB < FREE1 ? kring + 2 * TB + wv * QB : vring + TB + (wv * QB - FREE1);
      if (ntiles > 0) {
        // K(0) first: its address is ready, Q's take a division
        const auto pg0 = wave_page(0);
        issue_k(0, pg0);
        // lane: row wrow0 + lr + QRPI*i of instruction i, 16-byte chunk qcs.
        // Row -> (node, head) = (row / g, row % g) by one division, then
        // stepped by QRPI = (QRPI / g) * g + QRPI % g rows per instruction.
        constexpr int QRPI = 1024 / (D * 2);
        const int lr = lane / (D / 8), qcs = lane % (D / 8);
        const long long sn = p.q_stride_n, sh = p.q_stride_h;
        int row = wrow0 + lr;
        int qj = row % g;
        long long qoff = (long long)(row / g) * sn + (long long)qj * sh;
        const int dj = QRPI % g;
        const long long dstep = (long long)(QRPI / g) * sn + (long long)dj * sh, wrap = sn - (long long)g * sh;
        const bf16_t* q0p = (const bf16_t*)p.q + (long long)w.q0 * sn + (long long)(w.kvh * g) * sh;
        // (a wave with no valid row computes nothing and needs no Q)
#pragma unroll
        for (int i = 0; i < NQI && live; ++i) {
          // rows past the group's end read a valid row (node 0); their
          // results are never stored or merged
          dma16(q0p + (row < R ? qoff : 0ll) + 8 * (qcs ^ chunk_swizzle<D>(i * QRPI + lr)), qdst + i * 1024);
          row += QRPI;
          qoff += dstep;
          qj += dj;
          if (qj >= g) {
            qj -= g;
            qoff += wrap;
          }
        }
        issue_v(0, pg0);
      }
      if (1 < ntiles) issue_k(1, wave_page(1));
      // two-tile ranges (a 128-key window) whose Q staging leaves the V ring
      // free: V(1) goes out now, after K(1), instead of after the Q fragments
      const bool early_v1 = W * QB <= FREE1 && ntiles == 2;
      if (early_v1) issue_v(1, wave_page(1));
      // Q and K(0) have landed once at most V(0), K(1) (and V(1)) are outstanding
      wait_vmcnt_units<IPW, 3>((0 < ntiles ? 1 : 0) + (1 < ntiles ? 1 : 0) + (early_v1 ? 1 : 0));
      __builtin_amdgcn_s_barrier();  // every wave's share of K(0) is visible
      if (ntiles > 0) {
        const lds_char* qs = (const lds_char*)(uintptr_t)qdst;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
            qf[rb][ks] = *(const __attribute__((address_space(3))) bf16x8*)(qs + rb * 32 * D * 2 + koff[ks]);
      }
      // all Q fragments are in registers before the slots are refilled
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      // an empty range staged no Q; a following suffix-level call needs it
      if constexpr (!EPI) {
        if (ntiles == 0) load_q();
      }
      if (2 < ntiles) issue_k(2, wave_page(2));
      static_for<VST - 2>([&](auto j) {
        constexpr int st = decltype(j)::value - (VST - 2);
        if (st + VST - 1 < ntiles && !(early_v1 && st + VST - 1 == 1)) issue_v(st + VST - 1, wave_page(st + VST - 1));
        if (st + KST < ntiles) issue_k(st + KST, wave_page(st + KST));
      });
      auto pv_next = wave_page(VST - 1), pk_next = wave_page(KST);
      f32x16 sc[RB][2];
      if (live && ntiles > 0) {
        auto kf = kfrag_at(0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qk_ks(sc, kf, ks);
      }
      // Step s: wait until V(s) and K(s + 1) have landed.  V(s) was issued
      // after K(s + 1); the loads issued after V(s) may stay outstanding:
      // K(s + 2) and the V / K pairs of the VST - 2 following steps (those
      // tiles that exist).  The barrier makes every wave's share visible and
      // frees the slots of K(s) and V(s - 1).
      auto pstep_wait = [&](int it) {
        const int r = ntiles - 1 - it;
        const int kout = (r >= 2 ? 1 : 0) + min(r, VST - 2) + max(0, min(VST - 2, r - 2));
        __asm__ volatile("" ::: "memory");
        wait_vmcnt_units<IPW, MAXK>(kout);
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        if (it + VST - 1 < ntiles) issue_v(it + VST - 1, pv_next);
        if (it + KST < ntiles) issue_k(it + KST, pk_next);
        pv_next = wave_page(it + VST);
        pk_next = wave_page(it + KST + 1);
      };
      for (int it = 0; it + 1 < ntiles; ++it) {
        pstep_wait(it);
        if (live) pipelined_tile(sc, kfrag_at(it + 1), vfrag_at(it));
      }
      if (ntiles > 0) {
        // last tile: keys past kv_end (a partial tile) are masked
        pstep_wait(ntiles - 1);
        if constexpr (SEAM == 1) {
          // Every K slot and all V slots but V(ntiles - 1)'s are free now
          // (the barrier above): issue the suffix level's prologue tiles
          // (rows q0.. of k/v_suffix, the order of its own prologue) into
          // the ring rotated by ntiles, and its rows' tree-mask words, so
          // that they land during this last tile.
          if (p.mask_mode == MASK_TREE) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              if (rv[rb]) {
                const unsigned long long* mr = p.tree_mask + (long long)(w.q0 + n[rb]) * p.mask_words;
#pragma unroll
                for (int k = 0; k < kMaskRegWords; ++k) st.mreg[rb][k] = (k < p.mask_words) ? mr[k] : 0ull;
              }
          }
          const int nts = (w.nq + 63) >> 6;
          const long long stok = p.suf.stride_tok * 2;
          const long long soff = (long long)w.kvh * p.suf.stride_head * 2 + (long long)w.q0 * stok;
          auto issue_s = [&](const void* src, int j, unsigned slot) {
#pragma unroll
            for (int i = 0; i < IPW; ++i) {
              const int inst = wv * IPW + i;
              const int r = inst * RPI + lrow;
              dma16((const char*)src + soff + min(j * 64 + r, w.nq - 1) * stok + (cs ^ chunk_swizzle<D>(r)) * 16,
                    slot + inst * 1024);
            }
          };
          static_for<KST - 1>([&](auto jj) {
            constexpr int st_ = decltype(jj)::value - (KST - 1);
            if (st_ + VST - 1 >= 0 && st_ + VST - 1 < nts)
              issue_s(p.suf.v, st_ + VST - 1, vring + ((st_ + VST - 1 + ntiles) % VST) * TB);
            if (st_ + KST - 1 < nts) issue_s(p.suf.k, st_ + KST - 1, kring + ((st_ + KST - 1 + ntiles) % KST) * TB);
          });
        }
        if (live) {
          mask_scores(sc, kv_begin + (ntiles - 1) * 64, std::true_type{});
          finish_tile(sc, vfrag_at(ntiles - 1));
        }
      }
      if constexpr (SEAM == 1) {
        st.handoff = ntiles > 0;
        st.ring_off = ntiles;
      }
    } else {
      // ---- suffix level: masked tiles, skipped where no row sees a key ----
      // Issue order: step s issues V(s + VST - 1) then K(s + KST - 1); the
      // prologue plays steps -(KST - 1) .. -1.
      // (a fused item's prefix level already issued them: SEAM 2 with handoff)
      if (!(SEAM == 2 && st.handoff)) {
        static_for<KST - 1>([&](auto j) {
          constexpr int st_ = decltype(j)::value - (KST - 1);
          if (st_ + VST - 1 >= 0 && st_ + VST - 1 < ntiles) issue_v(st_ + VST - 1, wave_page(st_ + VST - 1));
          if (st_ + KST - 1 < ntiles) issue_k(st_ + KST - 1, wave_page(st_ + KST - 1));
        });
      }
      auto pk_next = wave_page(KST - 1), pv_next = wave_page(VST - 1);
      wait_vmcnt<0>();  // Q / mask loads and the first tiles (see above)

      // One step: wait for tile `it`, refill the K and V slots freed by tile
      // it-1, compute tile `it`.
      auto step = [&](int it) {
        // K(it) was issued before V(it); once V(it) has landed, the only loads
        // of this wave still outstanding are those issued after it: K(it + 1)
        // in the same step and the V and K tiles of the VST - 2 later steps
        // (those tiles that exist).  After the barrier every wave's share is
        // visible and the slots of tile it-1 are free.
        const int r = ntiles - 1 - it;
        const int kout = min(r, 1) + min(r, VST - 2) + max(0, min(r, VST - 1) - 1);
        __asm__ volatile("" ::: "memory");
        wait_vmcnt_units<IPW, MAXK>(kout);
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        if (it + VST - 1 < ntiles) issue_v(it + VST - 1, pv_next);
        if (it + KST - 1 < ntiles) issue_k(it + KST - 1, pk_next);
        pv_next = wave_page(it + VST);
        pk_next = wave_page(it + KST);

        const int kb = kv_begin + it * 64;
        if (!live || !tile_visible(kb)) return;
        compute_tile(kb, kfrag_at(it), vfrag_at(it), std::true_type{});
      };
      for (int it = 0; it < ntiles; ++it) step(it);
    }
  } else {
    // ============ register-staged tiles (fp8 e4m3fn -> bf16 in LDS) ============
    // Each thread loads 16 fp8 bytes (head dims 16s .. 16s + 15 of one key),
    // expands them to two bf16 chunks and stores those in the layout of the
    // direct-to-LDS rings (row-major, chunk c of key row r at position
    // c ^ swizzle(r)), so that K and V^T fragments are read exactly as there.
    wait_vmcnt<0>();  // Q / mask loads complete, visibly to the compiler (see above)
    constexpr int SEG = D / 16;                  // 16-byte fp8 segments per key row
    constexpr int NS = (64 * SEG + NT - 1) / NT;  // segments per thread and tile
    u32x4 kr[NS], vr[NS];                        // 16 fp8 elements each

    auto load_tile = [&](int kb) {
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int s_ = tid + i * NT;
        if (64 * SEG % NT == 0 || s_ < 64 * SEG) {
          const long long off = tok_off(min(kb + s_ / SEG, kv_end - 1)) + (s_ % SEG) * 16;
          kr[i] = *(const u32x4*)(kbase + off);
          vr[i] = *(const u32x4*)(vbase + off);
        }
      }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int s_ = tid + i * NT;
        if (64 * SEG % NT == 0 || s_ < 64 * SEG) {
          const int r = s_ / SEG, c0 = 2 * (s_ % SEG), sw = chunk_swizzle<D>(r);
          bf16_t* krow = &sm.st.k[buf][r * D];
          bf16_t* vrow = &sm.st.v[buf][r * D];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const u32x2 klo = fp8x4_to_bf16x4(kr[i][2 * h]), khi = fp8x4_to_bf16x4(kr[i][2 * h + 1]);
            const u32x2 vlo = fp8x4_to_bf16x4(vr[i][2 * h]), vhi = fp8x4_to_bf16x4(vr[i][2 * h + 1]);
            *(u32x4*)(krow + 8 * ((c0 + h) ^ sw)) = (u32x4){klo[0], klo[1], khi[0], khi[1]};
            *(u32x4*)(vrow + 8 * ((c0 + h) ^ sw)) = (u32x4){vlo[0], vlo[1], vhi[0], vhi[1]};
          }
        }
      }
    };

    // fragment offsets inside a tile (bytes), as for the direct-to-LDS rings
    unsigned koff[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) koff[ks] = (l32 * D + 8 * ((2 * ks + hh) ^ chunk_swizzle<D>(l32))) * 2;
    const int k16 = lane & 15;
    const int krow = 4 * hh + (k16 >> 2);
    const int dsub = 16 * ((lane >> 4) & 1) + 4 * (k16 & 3);
    unsigned voff0[MT], voff1[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int d = 32 * mt + dsub;
      voff0[mt] = (krow * D + 8 * ((d >> 3) ^ chunk_swizzle<D>(krow)) + (d & 7)) * 2;
      voff1[mt] = ((krow + 8) * D + 8 * ((d >> 3) ^ chunk_swizzle<D>(krow + 8)) + (d & 7)) * 2;
    }
    typedef __attribute__((address_space(3))) char lds_char;

    if (ntiles > 0) {
      load_tile(kv_begin);
      store_tile(0);
    }
    if (1 < ntiles) load_tile(kv_begin + 64);
    __syncthreads();
    auto step = [&](int it, auto masked_tile) {
      const int buf = it & 1;
      const int kb = kv_begin + it * 64;
      // tile it + 1 (loaded during the previous step) into the free buffer,
      // then the loads of tile it + 2, then the compute of tile it
      if (it + 1 < ntiles) store_tile(buf ^ 1);
      if (it + 2 < ntiles) load_tile(kb + 128);
      if (live) {
        const lds_char* kst = (const lds_char*)(uintptr_t)lds_address(&sm.st.k[buf][0]);
        const lds_char* vst = (const lds_char*)(uintptr_t)lds_address(&sm.st.v[buf][0]);
        auto kfrag = [&](int kt, int ks) -> bf16x8 {
          return *(const __attribute__((address_space(3))) bf16x8*)(kst + koff[ks] + kt * 32 * D * 2);
        };
        auto vfrag = [&](int mt, int ks) -> bf16x8 {
          typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vst + voff0[mt] + ks * 16 * D * 2));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vst + voff1[mt] + ks * 16 * D * 2));
          const u32x2 ulo = __builtin_bit_cast(u32x2, lo), uhi = __builtin_bit_cast(u32x2, hi);
          return __builtin_bit_cast(bf16x8, (u32x4){ulo[0], ulo[1], uhi[0], uhi[1]});
        };
        compute_tile(kb, kfrag, vfrag, masked_tile);
      }
      __syncthreads();
    };
    const int nfull = (kv_end - kv_begin) >> 6;
    for (int it = 0; it < nfull; ++it) step(it, std::false_type{});
    if (nfull < ntiles) step(nfull, std::true_type{});
  }

  if constexpr (!EPI) {
    // hand the state to the suffix level (bf16 keys and values): O in value
    // units, the running max in score units of unscaled keys
    if (live) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if (m_run[rb] != -INFINITY) m_run[rb] *= kscale;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) o[rb][mt] *= vscale;
      }
    }
    return;
  }

  // ---- epilogue ----
  // Final outputs (and the in-place merge) go through this wave's rows of the
  // ring, chunks swizzled by row as in the key tiles: each lane writes its
  // MFMA-layout part of the bf16 result, and the rows go out row by row (whole
  // rows per store instruction).  In place, the stored state (O_s, LSE_s),
  // read row by row in the prologue, goes in first and each lane merges its
  // part with this state (flashinfer.merge_state_in_place,
  // model/cascade_graph.py:58-60; both empty keeps the stored state).  The
  // sink (verification.py:173-176) scales the result.
  if (INPLACE || w.mode != MODE_PARTIAL) {
    static_assert(ROWS * D <= (KST + VST) * 64 * D, "the rows must fit the ring");
    __syncthreads();  // every wave is done with the key / value tiles
    bf16_t* reg = &sm.ring.k[0][0] + wv * RB * 32 * D;
    if constexpr (INPLACE) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < OIPB; ++i) {
          const int r = ORPI * i + lane / OCH;  // row in the 32-row block
          *(u32x4*)(reg + (32 * rb + r) * D + 8 * ((lane % OCH) ^ chunk_swizzle<D>(r))) = old_o[rb][i];
        }
    }
    if (live) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const float l_tot = l_run[rb] + xor32(l_run[rb], hh);
        const bool nonempty = l_tot > 0.f;
        // l_tot >= 1 when nonempty (the running max never exceeds the row's
        // maximum, whose term is then >= 1): the reciprocal is within 1 ulp
        const float inv = nonempty ? vscale * __builtin_amdgcn_rcpf(l_tot) : 0.f;
        const float lse_n = nonempty ? m_run[rb] * cn + logf(l_tot) : -INFINITY;
        float wa = 0.f, wb = inv, lse = lse_n;  // out = wa O_s + wb O
        if constexpr (INPLACE) {
          const float ol = p.lse_base2 ? old_lse[rb] * kLn2 : old_lse[rb];
          const float m = fmaxf(ol, lse_n);
          wa = 1.f;
          wb = 0.f;
          lse = ol;
          if (m != -INFINITY) {
            const float ea = __expf(ol - m), eb = __expf(lse_n - m);
            const float sum = ea + eb;  // in [1, 2]
            const float rs = __builtin_amdgcn_rcpf(sum);
            wa = ea * rs;
            wb = eb * rs * inv;
            lse = m + logf(sum);
          }
        }
        if (p.sinks) {
          const float sc = (lse == -INFINITY || !rv[rb]) ? 0.f : 1.f / (1.f + __expf(p.sinks[qh[rb]] - lse));
          wa *= sc;
          wb *= sc;
        }
        bf16_t* myrow = reg + (32 * rb + l32) * D + 4 * hh;
        u32x2 od[INPLACE ? MT : 1][4];  // all reads, then all writes: the reads issue back to back
        if constexpr (INPLACE) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
              od[mt][q4] = *(const u32x2*)(myrow + 8 * ((4 * mt + q4) ^ chunk_swizzle<D>(l32)));
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = o[rb][mt][4 * q4 + e] * wb;
            if constexpr (INPLACE) {
              v[0] += wa * bf16_lo(od[mt][q4][0]);
              v[1] += wa * bf16_hi(od[mt][q4][0]);
              v[2] += wa * bf16_lo(od[mt][q4][1]);
              v[3] += wa * bf16_hi(od[mt][q4][1]);
            }
            *(u32x2*)(myrow + 8 * ((4 * mt + q4) ^ chunk_swizzle<D>(l32))) =
                (u32x2){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          }
        if (p.lse && rv[rb] && hh == 0)
          p.lse[(long long)(w.q0 + n[rb]) * p.lse_stride_n + qh[rb]] = p.lse_base2 ? lse * kLog2e : lse;
      }
    }
    // (the reads below see this wave's own LDS writes above: a wave's LDS
    // operations complete in order).  The row addresses are recomputed from
    // an opaque copy of the lane index: reusing the prologue's would keep
    // them live across the tile loop.
    int olane;
    __asm__ volatile("v_mov_b32 %0, %1" : "=v"(olane) : "v"(lane));
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      RowWalk rw(wrow0 + 32 * rb + olane / OCH, ORPI, R, g, p.o_stride_n, p.o_stride_h);
      bf16_t* obase = (bf16_t*)p.o + (long long)w.q0 * p.o_stride_n + (long long)(w.kvh * g) * p.o_stride_h +
                      8 * (olane % OCH);
      u32x4 piece[OIPB];  // all reads first, then the stores
#pragma unroll
      for (int i = 0; i < OIPB; ++i) {
        const int r = ORPI * i + olane / OCH;
        piece[i] = *(const u32x4*)(reg + (32 * rb + r) * D + 8 * ((olane % OCH) ^ chunk_swizzle<D>(r)));
      }
#pragma unroll
      for (int i = 0; i < OIPB; ++i, rw.next())
        if (rw.valid()) *(u32x4*)(obase + rw.offset()) = piece[i];
    }
    return;
  }

  // partial state of a key chunk: normalised O and LSE to the workspace slot
  if (live) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const float l_tot = l_run[rb] + xor32(l_run[rb], hh);
      const bool nonempty = l_tot > 0.f;
      const float inv = nonempty ? vscale * __builtin_amdgcn_rcpf(l_tot) : 0.f;  // l_tot >= 1 (above)
      const float lse_r = nonempty ? m_run[rb] * cn + logf(l_tot) : -INFINITY;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) o[rb][mt] *= inv;
      // streaming stores: the merge launch reads each partial once, and
      // lines that leave L2 during the epilogue are not written back at the
      // kernel's end
      // (rows past the group's end are never merged: not stored)
      const int blk = RB * wv + rb;
      bf16_t* po = (bf16_t*)p.part_o + (long long)w.slot * ROWS * D;
      float* pl = p.part_lse + (long long)w.slot * ROWS + blk * 32 + l32;
      if (rv[rb]) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int pr = 0; pr < 2; ++pr)
            __builtin_nontemporal_store(image_piece(o[rb][mt], pr, 1.f),
                                        (u32x4*)(po + image_offset<D>(blk, mt, pr, lane)));
        if (hh == 0) __builtin_nontemporal_store(lse_r, pl);
      }
    }
  }
}

// Workgroup shapes (waves_per_block of the plan): 2 = two waves of 64 rows
// (one wave per SIMD, up to 512 registers), 4 = four waves of 32 rows and
// 8 = eight waves of 32 rows (two waves per SIMD, up to 256 registers).
template <int WPB>
struct Shape;
template <>
struct Shape<1> { static constexpr int W = 1, RB = 1, OCC = 1; };  // the in-place kind's 32-row workgroups
template <>
struct Shape<2> { static constexpr int W = 2, RB = 2, OCC = 1; };
template <>
struct Shape<4> { static constexpr int W = 4, RB = 1, OCC = 2; };
template <>
struct Shape<8> { static constexpr int W = 8, RB = 1, OCC = 2; };

// The prefix level (paged or contiguous, bf16 or fp8) and the suffix level
// (contiguous bf16, masked) share one launch; the item's src picks the body.
// Plans of each kind have a kernel of their own, so that no kind's register
// allocation carries another kind's path: KIND_SPLIT (prefix-chunk and suffix
// items), KIND_FUSED (no group split: SRC_BOTH and suffix items), KIND_INPLACE
// (suffix items merging into the stored output: the per-row local level of
// the drop-in runner), KIND_SEGMENTS (split plans over a two-segment
// contiguous prefix: SRC_PREFIX, SRC_PREFIX2 and suffix items).
// The in-place kind serves the drop-in runner's workgroups (rows x kv heads
// x 32-row blocks, one wave each): one wave per SIMD, so that its state, the
// stored output and the tree-mask words all stay in registers.
template <int D, int WPB, bool PAGED, bool FP8, int KIND>
__global__ __launch_bounds__(64 * WPB) __attribute__((amdgpu_waves_per_eu(KIND == KIND_INPLACE ? 1 : Shape<WPB>::OCC,
                                                                            KIND == KIND_INPLACE ? 1 : Shape<WPB>::OCC)))
void verify_attn_kernel(const VerifyItem* __restrict__ items, const int* __restrict__ prefix_len,
                        const VerifyParams p) {
  constexpr int W = Shape<WPB>::W, RB = Shape<WPB>::RB;
  using R = RingCfg<D, WPB>;
  __shared__ __attribute__((aligned(16))) VerifySmem<D, R::KST, R::VST, R::NPG> sm;
  const VerifyItem w = items[blockIdx.x];
  // prefix_len (p.prefix_len, preloaded like items): request 0's length is
  // fetched in the same round as the item, so a single-request dynamic plan
  // knows its key range when the item lands
  int len0 = 0;
  if (prefix_len) len0 = prefix_len[0];
  // Load the whole item and the prefix-level arguments in one round of
  // scalar loads (the compiler would otherwise fetch the fields used after
  // the mode test in later rounds): the Q loads and the first page ids
  // depend on both.
  __asm__ volatile("" ::"s"(w.kvh), "s"(w.qtile), "s"(w.kv_begin), "s"(w.kv_end), "s"(w.slot), "s"(w.q0), "s"(w.nq),
                   "s"(w.base), "s"(w.src));
  __asm__ volatile("" ::"s"(p.q), "s"(p.q_stride_n), "s"(p.q_stride_h), "s"(p.pre.k), "s"(p.pre.v),
                   "s"(p.pre.page_table), "s"(p.pre.stride_tok), "s"(p.pre.stride_head), "s"(p.pre.stride_page),
                   "s"(p.pre.log2_page), "s"(p.group), "s"(p.sm_scale_log2));
  if (w.mode == MODE_NOOP) return;
  VerifyState<RB, D / 32, D / 16> st;
  st.len0 = len0;
  if constexpr (KIND == KIND_INPLACE) {
    verify_body<D, W, RB, R::KST, R::VST, R::NPG, false, true, false, true, true, true>(p, w, p.suf, sm, st);
  } else if (KIND == KIND_SPLIT && w.src == SRC_PREFIX) {
    verify_body<D, W, RB, R::KST, R::VST, R::NPG, PAGED, false, FP8>(p, w, p.pre, sm, st);
  } else if (KIND == KIND_SEGMENTS && w.src != SRC_SUFFIX) {
    // a chunk of the contiguous prefix's first or second segment
    verify_body<D, W, RB, R::KST, R::VST, R::NPG, false, false, FP8>(p, w, w.src == SRC_PREFIX2 ? p.pre2 : p.pre,
                                                                      sm, st);
  } else if (w.src == SRC_SUFFIX) {
    verify_body<D, W, RB, R::KST, R::VST, R::NPG, false, true, false>(p, w, p.suf, sm, st);
  } else if constexpr (KIND == KIND_FUSED) {
    // SRC_BOTH: the group's whole visible prefix, then its suffix tree, in
    // one state, to the final output (no partial, no merge)
    verify_body<D, W, RB, R::KST, R::VST, R::NPG, PAGED, false, FP8, true, false, false, FP8 ? 0 : 1>(p, w, p.pre,
                                                                                                       sm, st);
    __syncthreads();  // every wave is done with the prefix tiles in the rings
    VerifyItem ws = w;
    ws.kv_begin = 0;
    ws.kv_end = w.nq;
    ws.base = w.q0;  // the request's suffix keys are rows q0.. of k/v_suffix
    verify_body<D, W, RB, R::KST, R::VST, R::NPG, false, true, false, false, true, false, FP8 ? 0 : 2>(p, ws, p.suf,
                                                                                                       sm, st);
  }
}

// ---------------------------------------------------------------------------
// Merge of one 32-row block `blk` of a group, head dims [32 mt, 32 mt + 32):
// the log-sum-exp merge of partial slots [slot0, slot0 + nslots)
// (flashinfer.merge_state_in_place semantics, generation/verification.py:
// 163-165) and the GPT-OSS sink (verification.py:173-176), written to O and
// LSE.  Lane l owns row l%32 and head dims 32mt + 8q4 + 4(l/32) + e; all
// partial loads (up to kMaxVerifySplits + 1 slots) are in flight at once.
// ---------------------------------------------------------------------------
template <int D, int ROWS>
__device__ __forceinline__ void merge_rows(const VerifyParams& p, int slot0, int nslots, int blk, int mt,
                                           int lane, int q0, int nq, int kvh, int qtile) {
  constexpr int B = kMaxVerifySplits + 1;
  const int l32 = lane & 31, hh = lane >> 5;
  const int g = p.group;
  const int row = qtile * ROWS + blk * 32 + l32;
  if (row >= nq * g) return;
  const int n = row / g, qh = kvh * g + (row - n * g);

  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  float mval = -INFINITY, wsum = 0.f;
  const long long slot_elems = (long long)ROWS * D;
  for (int s0 = 0; s0 < nslots; s0 += B) {
    const int cnt = min(B, nslots - s0);
    float ls[B];
    u32x4 v[B][2];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      ls[b] = -INFINITY;
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) v[b][pr] = (u32x4){0u, 0u, 0u, 0u};
      if (b < cnt) {
        const long long s = slot0 + s0 + b;
        const float* pl = p.part_lse + s * ROWS + blk * 32 + l32;
        ls[b] = *pl;
        const bf16_t* po = (const bf16_t*)p.part_o + s * slot_elems;
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) v[b][pr] = *(const u32x4*)(po + image_offset<D>(blk, mt, pr, lane));
      }
    }
    float bm = -INFINITY;
#pragma unroll
    for (int b = 0; b < B; ++b) bm = fmaxf(bm, ls[b]);
    const float nm = fmaxf(mval, bm);
    if (nm == -INFINITY) continue;  // nothing visible so far
    const float f = (mval == -INFINITY) ? 0.f : __expf(mval - nm);
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] *= f;
    wsum *= f;
#pragma unroll
    for (int b = 0; b < B; ++b) {
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
  bf16_t* orow = (bf16_t*)p.o + (long long)(q0 + n) * p.o_stride_n + (long long)qh * p.o_stride_h;
  store_row_block32(orow + 32 * mt, acc, sc, hh);
  if (p.lse && mt == 0 && hh == 0)
    p.lse[(long long)(q0 + n) * p.lse_stride_n + qh] = p.lse_base2 ? lse * kLog2e : lse;
}

// Merge launch: one single-wave workgroup per (group, 32-row block, 32-wide
// head-dim block mt), so that the partial loads spread over every CU.  The
// grid is (merges rounded up to a multiple of 8) x (D / 32): workgroup (m, mt)
// has linear index m + nm8 * mt, so merge m stays on XCD m % 8, the XCD of its
// partials.
template <int D, int ROWS>
__global__ __launch_bounds__(64) void verify_merge_kernel(const VerifyMerge* __restrict__ merges, const VerifyParams p) {
  const int mi = blockIdx.x, mt = blockIdx.y;
  // the arguments in one round of scalar loads, then the whole record in one
  __asm__ volatile("" ::"s"(merges), "s"(p.num_merges), "s"(p.part_o), "s"(p.part_lse), "s"(p.o),
                   "s"(p.o_stride_n), "s"(p.o_stride_h), "s"(p.lse), "s"(p.lse_stride_n), "s"(p.group),
                   "s"(p.sinks), "s"(p.lse_base2));
  if (mi >= p.num_merges) return;
  const VerifyMerge m = merges[mi];
  __asm__ volatile("" ::"s"(m.kvh), "s"(m.qtile), "s"(m.slot0), "s"(m.nslots), "s"(m.q0), "s"(m.nq), "s"(m.blk));
  if (m.nslots == 0) return;  // padding
  merge_rows<D, ROWS>(p, m.slot0, m.nslots, m.blk, mt, threadIdx.x, m.q0, m.nq, m.kvh, m.qtile);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int D, int WPB, bool PAGED, bool FP8, int KIND>
static hipError_t launch_verify_t(const VerifyParams& p, int nitems, hipStream_t s) {
  hipLaunchKernelGGL((verify_attn_kernel<D, WPB, PAGED, FP8, KIND>), dim3(nitems), dim3(64 * WPB), 0, s, p.items, p.prefix_len, p);
  return hipGetLastError();
}

template <int D, int WPB, int KIND>
static hipError_t launch_verify_k(const VerifyParams& p, bool paged, bool fp8, int nitems, hipStream_t s) {
  if (fp8)
    return paged ? launch_verify_t<D, WPB, true, true, KIND>(p, nitems, s)
                 : launch_verify_t<D, WPB, false, true, KIND>(p, nitems, s);
  return paged ? launch_verify_t<D, WPB, true, false, KIND>(p, nitems, s)
               : launch_verify_t<D, WPB, false, false, KIND>(p, nitems, s);
}

template <int D, int WPB>
static hipError_t launch_verify_w(const VerifyParams& p, bool paged, bool fp8, int kind, int nitems, hipStream_t s) {
  // in-place plans (the drop-in runner's) read no prefix and are planned with
  // one wave per workgroup, a shape no other kind has
  if constexpr (WPB == 1) {
    return kind == KIND_INPLACE ? launch_verify_t<D, 1, false, false, KIND_INPLACE>(p, nitems, s)
                                : hipErrorInvalidValue;
  } else {
    if (kind == KIND_INPLACE) return hipErrorInvalidValue;
    if (kind == KIND_FUSED) return launch_verify_k<D, WPB, KIND_FUSED>(p, paged, fp8, nitems, s);
    // two-segment prefixes are contiguous
    if (kind == KIND_SEGMENTS)
      return paged ? hipErrorInvalidValue
             : fp8 ? launch_verify_t<D, WPB, false, true, KIND_SEGMENTS>(p, nitems, s)
                   : launch_verify_t<D, WPB, false, false, KIND_SEGMENTS>(p, nitems, s);
    return launch_verify_k<D, WPB, KIND_SPLIT>(p, paged, fp8, nitems, s);
  }
}

hipError_t launch_verify_attention(const VerifyParams& p, int head_dim, int waves, bool paged, bool fp8, int kind,
                                   int nitems, hipStream_t s) {
  if (nitems <= 0) return hipSuccess;
  if (kind != KIND_SPLIT && kind != KIND_FUSED && kind != KIND_INPLACE && kind != KIND_SEGMENTS)
    return hipErrorInvalidValue;
  if (head_dim == 128) {
    if (waves == 1) return launch_verify_w<128, 1>(p, paged, fp8, kind, nitems, s);
    if (waves == 2) return launch_verify_w<128, 2>(p, paged, fp8, kind, nitems, s);
    if (waves == 4) return launch_verify_w<128, 4>(p, paged, fp8, kind, nitems, s);
    if (waves == 8) return launch_verify_w<128, 8>(p, paged, fp8, kind, nitems, s);
  } else if (head_dim == 64) {
    if (waves == 1) return launch_verify_w<64, 1>(p, paged, fp8, kind, nitems, s);
    if (waves == 2) return launch_verify_w<64, 2>(p, paged, fp8, kind, nitems, s);
    if (waves == 4) return launch_verify_w<64, 4>(p, paged, fp8, kind, nitems, s);
    if (waves == 8) return launch_verify_w<64, 8>(p, paged, fp8, kind, nitems, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_verify_merge(const VerifyParams& p, int head_dim, int rows, int nmerges, hipStream_t s) {
  if (nmerges <= 0) return hipSuccess;
  if (p.num_merges != nmerges) return hipErrorInvalidValue;
  const int nm8 = (nmerges + 7) & ~7;
  const dim3 grid((unsigned)nm8, (unsigned)(head_dim / 32)), block(64);
  if (head_dim == 128 && rows == 128) hipLaunchKernelGGL((verify_merge_kernel<128, 128>), grid, block, 0, s, p.merges, p);
  else if (head_dim == 128 && rows == 256) hipLaunchKernelGGL((verify_merge_kernel<128, 256>), grid, block, 0, s, p.merges, p);
  else if (head_dim == 64 && rows == 128) hipLaunchKernelGGL((verify_merge_kernel<64, 128>), grid, block, 0, s, p.merges, p);
  else if (head_dim == 64 && rows == 256) hipLaunchKernelGGL((verify_merge_kernel<64, 256>), grid, block, 0, s, p.merges, p);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Library-owned partial-state workspace of d2sd_cascade_run_noalloc: one
// static device array per GPU (kVerifyScratchBytes), held until the process
// ends.  In host code `scratch` names a host-side stand-in, so its device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and only that address is ever handed to kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[kVerifyScratchBytes];

hipError_t verify_scratch(void** ptr) {
  static std::mutex mu;
  static std::vector<void*> per_device;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)per_device.size() <= dev) per_device.resize(dev + 1, nullptr);
  if (!per_device[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    per_device[dev] = p;
  }
  *ptr = per_device[dev];
  return hipSuccess;
}

}  // namespace d2sd
