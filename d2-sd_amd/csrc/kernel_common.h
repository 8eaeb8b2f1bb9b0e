// Device helpers shared by the gfx950 attention kernels (attention.hip,
// verify_attention.hip): vector types, bf16 packing, fp8 expansion, the
// direct global->LDS copy and explicit vmcnt waits.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace d2sd {

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N-1>{})
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef __bf16 bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Lazy rescaling: the running max used for exponentiation may trail the true
// row max by up to 2^kRescaleSlack before O and l are rescaled.
constexpr float kRescaleSlack = 8.0f;
// Tree-mask words held in registers per row (rows of up to 128 nodes); later
// words are read from the (cached) mask row when their tile comes up.
constexpr int kMaskRegWords = 2;

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

// Element offset, inside one partial slot, of the 8 values (q4 = 2pr and
// 2pr + 1 of block mt) that lane `lane` of 32-row block `blk` holds: the
// accumulator register image in 16-byte lane pieces, so that every partial
// store / load is one contiguous 1 KB wave access.  (8-byte pieces took twice
// the load instructions in the merge, whose time follows their count: 4.60 vs
// 4.15 us per merge launch for a 150-node Qwen3-8B tree over 4096 keys.)
template <int D>
__device__ __forceinline__ int image_offset(int blk, int mt, int pr, int lane) {
  return ((blk * (D / 32) + mt) * 2 + pr) * 512 + 8 * lane;
}

// Values 8pr .. 8pr + 7 of an accumulator block (head dims 8q4 + 4hh + 0..3
// for q4 = 2pr, 2pr + 1) as one 16-byte image piece, each scaled by sc.
__device__ __forceinline__ u32x4 image_piece(const f32x16& o, int pr, float sc) {
  return (u32x4){pack_bf16x2(o[8 * pr] * sc, o[8 * pr + 1] * sc), pack_bf16x2(o[8 * pr + 2] * sc, o[8 * pr + 3] * sc),
                 pack_bf16x2(o[8 * pr + 4] * sc, o[8 * pr + 5] * sc), pack_bf16x2(o[8 * pr + 6] * sc, o[8 * pr + 7] * sc)};
}

// Store of one row's 32 head dims from a lane pair: lane l (row l % 32,
// hh = l / 32) holds acc[4q + e] = dim 8q + 4hh + e, q < 4, e < 4, scaled by
// sc.  The pair exchanges halves (v_permlane32_swap) so that lane hh writes
// dims 16hh .. 16hh + 15 as two 16-byte stores instead of four 8-byte ones
// (merge launch for a 150-node Qwen3-8B tree over 4096 keys: 4.17 -> 4.04
// us).  Both lanes of a pair must be active.
__device__ __forceinline__ void store_row_block32(bf16_t* dst, const float (&acc)[16], float sc, int hh) {
  unsigned wd[4][2];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    wd[q][0] = pack_bf16x2(acc[4 * q] * sc, acc[4 * q + 1] * sc);
    wd[q][1] = pack_bf16x2(acc[4 * q + 2] * sc, acc[4 * q + 3] * sc);
  }
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    // after the swaps lane hh holds both halves of chunk c + 2hh
    const auto a0 = __builtin_amdgcn_permlane32_swap(wd[c][0], wd[c + 2][0], false, false);
    const auto a1 = __builtin_amdgcn_permlane32_swap(wd[c][1], wd[c + 2][1], false, false);
    *(u32x4*)(dst + 8 * (c + 2 * hh)) = (u32x4){a0[0], a1[0], a0[1], a1[1]};
  }
}

// fp8 e4m3fn (OCP) -> bf16, exact: every finite e4m3fn value is a bf16 value.
// Bytes b0..b3 of w -> 4 bf16 in a u32x2, by the gfx950 converter
// v_cvt_scalef32_pk_bf16_fp8 at scale 1 (word select 0: bytes 0, 1; 1: bytes
// 2, 3).  Checked on the GPU against the exact value of all 254 finite bytes
// (NaN bytes give NaN); one instruction per pair instead of ten VALU
// operations of an expansion through fp16 (attention launch of 32 Qwen3-32B
// requests over 8192-key fp8 prefixes: 1508 -> 1271 us).
__device__ __forceinline__ u32x2 fp8x4_to_bf16x4(unsigned w) {
  return (u32x2){__builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, false)),
                 __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, true))};
}

// One global_load_lds_dwordx4: lane l copies 16 bytes from `src` to LDS byte
// address lds_addr + 16*l (lds_addr wave-uniform, passed through M0, which the
// statement declares clobbered).  Issued as inline asm so that the compiler
// does not track these LDS writes: its own tracking waits for every
// outstanding DMA (vmcnt(0)) before LDS reads, which would drain the whole
// prefetch ring each tile.  Completion is enforced explicitly (wait_vmcnt +
// s_barrier).  The loads are non-temporal (nt): a key / value tile is read by
// the workgroups of one launch at about the same time and never again, so it
// should not displace the partial states that the merge reads back from L2.
__device__ __forceinline__ void dma16(const void* src, unsigned lds_addr) {
  __asm__ volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off nt"
      :
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(src)
      : "memory", "m0");
}

// The same with a wave-uniform base: lane l copies 16 bytes from
// sbase + voff (voff per lane).  sbase and lds_addr must be wave-uniform;
// they are moved to scalar registers here (free when the compiler already
// holds them there).
__device__ __forceinline__ void dma16s(const void* sbase, unsigned voff, unsigned lds_addr) {
  // (readfirstlane returns int: widen through unsigned, never sign-extend)
  const unsigned long long b = (unsigned long long)sbase;
  const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((unsigned)(b >> 32));
  const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((unsigned)b);
  const unsigned long long sb = ((unsigned long long)hi << 32) | (unsigned long long)lo;
  __asm__ volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2 nt"
      :
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"((const void*)sb)
      : "memory", "m0");
}

__device__ __forceinline__ unsigned lds_address(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// s_waitcnt with vmcnt <= N and no wait on the other counters (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// XOR swizzle of 16-byte chunks in a key row (row pitch 256 B for D = 128,
// 128 B for D = 64), chosen so that both LDS read patterns of a tile are free
// of bank conflicts (LDS serves 256 bytes per pass):
//  * K fragments, ds_read_b128: 16 lanes read one logical chunk of 16
//    consecutive rows -> the swizzle is a bijection over any 16 aligned rows
//    (for D = 64, over the 8 rows of each parity, which share a 256-byte line
//    pair position);
//  * V^T fragments, ds_read_b64_tr_b16: 32 lanes read 4 consecutive logical
//    chunks (4m .. 4m+3) of 4 consecutive rows 4a .. 4a+3 -> those rows'
//    swizzles differ in the bits above the low two (bits 2-3 for D = 128,
//    bit 2 between rows of equal parity for D = 64).
// The plain `chunk ^ row` swizzle satisfies only the first and leaves the
// transposed reads 4-way conflicted (measured: 63 vs 185 B/clk per CU).
template <int D>
__device__ __forceinline__ int chunk_swizzle(int row) {
  return D == 128 ? (((row & 3) << 2) | ((row >> 2) & 3)) : ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
}

}  // namespace d2sd
