// Where the attention kernels read the paged cache: the position -> block -> element -> byte
// arithmetic and the chunk geometry, as __host__ __device__ functions. The kernels call these
// for every K/V address they form, and the host-side address walk (kv_reach.hip) calls the same
// ones to enumerate every address a launch would read, so a CPU test can check that each stays
// inside the cache. Both fault classes this guards against -- element offsets used as byte
// offsets for fp8 codes, and indices past a staged buffer -- live in this arithmetic.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "ayaka_hip_internal.h"

namespace ayk {

#define AYK_HD __host__ __device__ __forceinline__
#ifndef AYK_F32_WIDE_GC
#define AYK_F32_WIDE_GC 4
#endif

AYK_HD int imin(int a, int b) { return a < b ? a : b; }
AYK_HD int imax(int a, int b) { return a > b ? a : b; }

// High 32 bits of a 32 x 32-bit product (v_mul_hi_u32 on the device).
AYK_HD uint32_t mul_hi_u32(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umulhi(a, b);
#else
  return (uint32_t)(((uint64_t)a * b) >> 32);
#endif
}

// Product of the low 24 bits of each operand, low 32 bits of it (the full-rate
// v_mul_u32_u24 on the device).
AYK_HD uint32_t mul_u24(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul24(a, b);
#else
  return (a & 0xffffffu) * (b & 0xffffffu);
#endif
}

// Block of position t (0 <= t < 2^31) for any block size: a multiply-high division by the
// host's magic number, q = (umulhi(t, m) + t) >> l with l = ceil(log2 bs) and
// m = floor(2^32 (2^l - bs) / bs) + 1 (a power of two has m = 1: a shift). The sum stays
// below 2^32 because umulhi(t, m) < t < 2^31.
AYK_HD int block_of(const AttnParams& p, int t) {
  return (int)((mul_hi_u32((uint32_t)t, p.bs_magic) + (uint32_t)t) >> p.bs_shift);
}

// The staged table entry of block id b: the element offset of its block, or of the padding
// block 0 for an id outside the pool (bad metadata reads block 0 rather than faulting). The
// host checks that every offset in the pool fits 32 bits.
AYK_HD uint32_t table_entry(const AttnParams& p, int b) {
  return ((unsigned)b < (unsigned)p.num_blocks) ? (uint32_t)b * (uint32_t)p.block_stride : 0u;
}

// Element offset of position t in the cache, from the staged table segment that starts at
// block b0: its block's offset plus (t mod block size) x token stride, the products on the
// 24-bit multiplier (the block index is below the table width and the token stride below
// 2^24: the host refuses wider tables and strides).
AYK_HD uint32_t kv_offset(const AttnParams& p, const uint32_t* s_tbl, int b0, int t, uint32_t token_stride) {
  const int b = block_of(p, t);
  const uint32_t r = (uint32_t)t - mul_u24((uint32_t)b, (uint32_t)p.block_size);
  return s_tbl[b - b0] + mul_u24(r, token_stride);
}

// Bytes from a cache's base to element `elem`: 2-byte elements, or 1-byte fp8 codes.
template <bool KV8>
AYK_HD int64_t kv_bytes_of(int64_t elem) {
  return KV8 ? elem : 2 * elem;
}

// Bytes one K/V load reads: 8 elements, 16 bytes of fp16/bf16 or 8 of fp8 codes.
template <bool KV8>
constexpr int kv_load_bytes() {
  return KV8 ? 8 : 16;
}

// Positions of one staged table segment for chunks of `ch` positions: at most kTableCap
// blocks, whatever the segment's first position's offset within its block.
AYK_HD int segment_positions(const AttnParams& p, int ch) { return ((kTableCap - 1) * p.block_size / ch) * ch; }

// Position read by load j of chunk ci of segment [s0, s1) for a lane at token r of each load
// of `tpl` tokens: past the segment's end it reads the last position again (weight 0 later).
AYK_HD int chunk_position(int s0, int s1, int ci, int ch, int j, int tpl, int r) {
  return imin(s0 + ci * ch + j * tpl + r, s1 - 1);
}

// The last chunk of a segment of nch chunks that slice `slice` of `ws` waves takes (it takes
// chunks slice, slice + ws, ...); below `slice` when the slice has none.
AYK_HD int last_chunk_of_slice(int nch, int slice, int ws) { return slice + (nch - 1 - slice) / ws * ws; }

// --- chunk geometry of each kernel ------------------------------------------------------------

// Decode (matrix-core kernel): 16-position MFMA tiles, SUB of them per chunk, so that a wave
// keeps about as many bytes in flight as a 16-bit tile of head_dim 128: fp8 loads and head_dim
// 64 carry half of that per tile (two tiles), fp8 at head_dim 64 a quarter (four); at head_dim
// 256 two fp8 tiles' loads do not fit the registers (they spilled), one does.
constexpr int decode_tiles_per_chunk(int d, bool kv8) { return d == 64 ? (kv8 ? 4 : 2) : (kv8 && d <= 128 ? 2 : 1); }
constexpr int decode_tile_positions() { return 16; }
// 8-element pieces per position, positions per load instruction (one piece per lane).
constexpr int pieces_per_position(int d) { return d / 8; }
constexpr int positions_per_load(int d) { return 64 / pieces_per_position(d); }

// Decode (DPP kernel): two loads per lane per chunk.
constexpr int dpp_loads_per_chunk() { return 2; }

// Decode over fp32 caches: 4 floats (16 bytes) per lane, so D / 4 lanes per position, and four
// token slots per lane and chunk; with more than AYK_F32_WIDE_GC query heads per wave 8 floats
// (two adjacent 16-byte loads) per lane, D / 8 lanes per position and two token slots, which
// halves the lane reductions per byte (measured: 8 heads per wave 1060 -> 987 us at C5's shape,
// 4 heads 321 -> 351 us at C3's, so 4 heads keep the narrow rows).
constexpr int f32_floats_per_lane(int gc) { return AYK_F32_WIDE_GC < gc ? 8 : 4; }
constexpr int f32_lanes_per_position(int d, int gc) { return d / f32_floats_per_lane(gc); }
constexpr int f32_loads_per_chunk(int gc) { return f32_floats_per_lane(gc) == 8 ? 2 : 4; }

// Multi-row kernel: 64-position chunks, or 32 at head_dim 256 with 1 or 2 waves per pair group
// (a 64-position stage there took 133 KB of LDS and left one wave per SIMD).
constexpr int prefill_chunk_positions(int d, int waves_per_group) { return d == 256 && waves_per_group <= 2 ? 32 : 64; }

// Element offsets, from the head's base, of the `n` consecutive positions t .. t + n - 1 of a
// multi-row chunk that one thread loads (its piece `piece`), past the segment's last position
// s1 - 1 reading that one. With a block size that is a multiple of n (uniform across the
// launch; t is then a multiple of n too) the positions share a block: one table lookup.
template <int N>
AYK_HD void prefill_offsets(const AttnParams& p, const uint32_t* s_tbl, int b0, int t, int s1, int piece,
                            uint32_t token_stride, uint32_t (&off)[N]) {
  const uint32_t bs = (uint32_t)p.block_size;
  auto offset_of = [&](int pos) {
    const int b = block_of(p, pos);
    const uint32_t r = (uint32_t)pos - mul_u24((uint32_t)b, bs);
    return s_tbl[b - b0] + mul_u24(r, token_stride) + piece * 8;
  };
  if (bs % N == 0) {
    const int last = s1 - 1;
    const uint32_t o0 = offset_of(imin(t, last));
#pragma unroll
    for (int u = 0; u < N; ++u) off[u] = o0 + (uint32_t)imin(u, imax(last - t, 0)) * token_stride;
  } else {
#pragma unroll
    for (int u = 0; u < N; ++u) off[u] = offset_of(imin(t + u, s1 - 1));
  }
}

}  // namespace ayk
