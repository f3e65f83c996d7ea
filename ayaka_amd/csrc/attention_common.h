// Device helpers shared by the paged-attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "ayaka_hip_internal.h"
#include "kv_address.h"

namespace ayk {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
// Most waves in one workgroup (one per virtual head).
constexpr int kMaxWaves = kMaxWavesPerGroup;

template <bool BF16>
struct Elem;

template <>
struct Elem<true> {
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
  // Round to nearest even, NaN kept quiet (what torch's float -> bfloat16 does).
  static __device__ __forceinline__ uint32_t round(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
  }
};

template <>
struct Elem<false> {
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
  static __device__ __forceinline__ uint32_t round(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  }
};

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of LPT lanes (8, 16 or 32); every lane gets its group's sum.
template <int LPT>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]: lane ^ 1
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]: lane ^ 2
  x += dpp<0x141>(x);  // row_half_mirror: the other quad of the 8
  if constexpr (LPT >= 16) x += dpp<0x140>(x);  // row_mirror: the other 8 of the 16
  if constexpr (LPT >= 32) x += __shfl_xor(x, 16);
  return x;
}

// The maximum over lanes l, l ^ 16, l ^ 32 and l ^ 48 (one value per 16-lane column), through
// gfx950's lane-swap instructions (no LDS round trip, unlike a bpermute): v_permlane16_swap
// exchanges the odd 16-lane rows of its first operand with the even rows of its second, so
// with x in both, the two results hold x[l] and x[l ^ 16] in some order; v_permlane32_swap
// does the same with the wave's halves.
__device__ __forceinline__ float column_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier that orders LDS only. __syncthreads() also waits for every
// outstanding global load, which would drain a software pipeline of prefetched
// chunks at each step; here loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// K/V are read exactly once per call: nontemporal loads keep them from displacing
// reusable lines and stream measurably faster on MI355X than plain loads.
__device__ __forceinline__ u32x4 stream_load(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// ---------------------------------------------------------------------------
// fp8 KV caches (codec "fp8_e4m3": OCP e4m3, the float8_e4m3fn format).
//
// Two codes of a word (its low or high half) to a packed pair of the compute
// type, in one v_cvt_scalef32_pk_{bf16,f16}_fp8 with scale 1: every e4m3 value
// (|x| <= 448, at most 4 significant bits, down to 2^-9) is exactly a bf16 and
// an fp16 value, so the conversion loses nothing. The NaN code decodes to NaN.
template <bool BF16, bool HIGH>
__device__ __forceinline__ uint32_t e4m3_pair(uint32_t word) {
  if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, HIGH));
  else return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, HIGH));
}

// Address of element `elem` of a cache: 2-byte elements, or 1-byte fp8 codes.
template <bool KV8>
__device__ __forceinline__ const uint16_t* kv_at(const uint16_t* base, int64_t elem) {
  return reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(base) + kv_bytes_of<KV8>(elem));
}

// Raw loads and decoding are separate, so prefetched chunks stay in flight: a
// decode at the load would make the wave wait for the data right away.
// The 8 elements at element offset `off` from `base` (see kv_at) as loaded:
// 16 bytes of fp16/bf16, or 8 bytes of fp8 codes. Nontemporal (STREAM) where
// the cache is read once per call (decode); plain where workgroups share it
// (the multi-row kernel's tiles of one request and head read the same chunks).
template <bool KV8>
struct KvRaw {
  typedef u32x4 T;
};
template <>
struct KvRaw<true> {
  typedef u32x2 T;
};

template <bool KV8, bool STREAM = true>
__device__ __forceinline__ typename KvRaw<KV8>::T load_kv_raw(const uint16_t* base, uint32_t off) {
  const auto* p8 = reinterpret_cast<const uint8_t*>(base) + kv_bytes_of<KV8>(off);
  typedef typename KvRaw<KV8>::T T;
  if constexpr (STREAM) return __builtin_nontemporal_load(reinterpret_cast<const T*>(p8));
  else return *reinterpret_cast<const T*>(p8);
}

// Loaded elements as 8 packed compute-type values (4 pairs).
template <bool KV8, bool BF16>
__device__ __forceinline__ u32x4 kv_pairs(typename KvRaw<KV8>::T w) {
  if constexpr (KV8)
    return u32x4{e4m3_pair<BF16, false>(w.x), e4m3_pair<BF16, true>(w.x), e4m3_pair<BF16, false>(w.y),
                 e4m3_pair<BF16, true>(w.y)};
  else
    return w;
}

// Loaded elements as 8 fp32 values (fp8 codes decode straight to fp32).
template <bool KV8, bool BF16>
__device__ __forceinline__ void kv_floats(typename KvRaw<KV8>::T w, float (&f)[8]) {
  if constexpr (KV8) {
    const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w.x, false);
    const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w.x, true);
    const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8((int)w.y, false);
    const f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8((int)w.y, true);
    f[0] = a[0]; f[1] = a[1]; f[2] = b[0]; f[3] = b[1];
    f[4] = c[0]; f[5] = c[1]; f[6] = d[0]; f[7] = d[1];
  } else {
    using E = Elem<BF16>;
    f[0] = E::lo(w.x); f[1] = E::hi(w.x);
    f[2] = E::lo(w.y); f[3] = E::hi(w.y);
    f[4] = E::lo(w.z); f[5] = E::hi(w.z);
    f[6] = E::lo(w.w); f[7] = E::hi(w.w);
  }
}

// The (row, head group, partition) a workgroup serves. The grid is flat and
// workgroups are handed to the 8 XCDs round-robin by linear id, so the order
// decides the balance across XCDs:
//  * with a work list (v2 planned on the host), workgroup id covers item
//    id / groups, head group id % groups: consecutive items -- the list holds
//    only partitions with tokens, longest first -- go to different XCDs;
//  * without one, the grid is dense over rows x groups x partitions with the
//    partition fastest, so the partitions of one row spread over every XCD
//    instead of all landing on XCD row % 8.
struct WgCoord {
  int row;
  int group;
  int part;
  int psize;  // v2: the partition size (the launch's, or the one staged for this step)
};

// The v2 partition size: the launch's, or the one staged on the device for this step.
__device__ __forceinline__ int partition_size_of(const AttnParams& p) {
  return p.staged ? p.staged[0] : p.partition_size;
}

// A workgroup's (row, head group, partition). With staged parameters the grid is an
// upper bound: workgroups past the staged item count get row -1 and do nothing. The item's
// entry (one exists for every workgroup of the grid: the list's capacity bounds it), the
// staged count and the staged partition size are read unconditionally -- the last two from
// a valid stand-in address when nothing is staged -- so they cost one round trip together.
__device__ __forceinline__ WgCoord wg_coord(const AttnParams& p, int groups, bool split) {
  int id = blockIdx.x;
  if (split && p.work) {
    const int item = id / groups;
    const int32_t* st = p.staged ? p.staged : p.work;
    const int row = p.work[2 * item], part = p.work[2 * item + 1];
    const int size = st[0], count = st[1];
    // a select, not an early return: the row and the count are then needed together
    const bool past = p.staged && item >= count;
    return WgCoord{past ? -1 : row, id % groups, part, p.staged ? size : p.partition_size};
  }
  const int parts = split ? p.max_partitions : 1;
  const int part = id % parts;
  id /= parts;
  const int size = *(p.staged ? p.staged : p.kv_lengths);  // a valid stand-in address without staging
  return WgCoord{id / groups, id % groups, part, split ? (p.staged ? size : p.partition_size) : 0};
}

// The request of row `row` (row n is request n without a request_of_row list).
__device__ __forceinline__ int row_request(const AttnParams& p, int row) {
  if (p.request_of_row) return p.request_of_row[row];  // uniform: decode launches load nothing
  return row;
}

// Length of row `row`'s context (request `req`), clamped so no read leaves the table. The
// row's position is read unconditionally (from a valid stand-in address when rows have none)
// beside the request's length.
__device__ __forceinline__ int row_length(const AttnParams& p, int row, int req) {
  const int pos = *(p.positions ? p.positions + row : p.kv_lengths);
  int len = p.kv_lengths[req];
  if (len > 0 && p.positions) len = min(len, pos + 1);
  return max(0, min(len, p.max_len));
}

// Length of row `row`'s context and its request, clamped so no read leaves the table.
// The row's position and request are read unconditionally (from a valid stand-in address
// when a table is absent) and ahead of the request's length, so the lookups overlap instead
// of each waiting behind a branch.
__device__ __forceinline__ void row_context(const AttnParams& p, int row, int& req, int& len) {
  const int pos = *(p.positions ? p.positions + row : p.kv_lengths);
  const int r = *(p.request_of_row ? p.request_of_row + row : p.kv_lengths);
  req = p.request_of_row ? r : row;
  len = p.kv_lengths[req];
  if (len > 0 && p.positions) len = min(len, pos + 1);
  len = max(0, min(len, p.max_len));
}

// Running-max sentinel: below any real score yet finite, so exp2(sentinel - m) is 0
// for a real m and 1 when nothing has been seen, and no -inf - -inf NaN can arise.
constexpr float kNoScore = -1.0e30f;
// How far (log2 units) the running max may trail a chunk's max before the
// accumulators are rescaled: weights stay below 2^8, far inside fp32.
constexpr float kRescaleSlack = 8.0f;

// Index of the first partial (partition 0) of (row, head), which has np partitions.
// By default the partials are [n_rows, num_heads, max_partitions]; with staged
// parameters the rows are packed: row r's partials start at slot staged[2 + r] (the
// host's prefix sum of the rows' partition counts), head-major within the row, so a
// launch needs as many slots as its work list holds items, not rows x max_partitions.
__device__ __forceinline__ int64_t partial_index(const AttnParams& p, int row, int head, int np) {
  return p.staged ? (int64_t)p.staged[2 + row] * p.num_heads + (int64_t)head * np
                  : ((int64_t)row * p.num_heads + head) * p.max_partitions;
}

// Write one head's merged state from lane c (its 8 elements): the rounded
// output (v1, or v2 for a row whose context is one partition: nothing to merge,
// so it rounds exactly what v1 rounds) or the normalised partial and its (m, l)
// (v2 partition `part` of `np`). Both carry the value scale, so the merges of
// partials need none.
template <int D, bool BF16, bool SPLIT>
__device__ __forceinline__ void store_head(const AttnParams& p, int row, int part, int np, int head, int c,
                                           const float (&o)[8], float m, float l) {
  using E = Elem<BF16>;
  const float inv = (l > 0.f ? 1.0f / l : 0.f) * p.v_scale;  // exact at v_scale 1
  const int64_t head_row = (int64_t)row * p.num_heads + head;
  if (SPLIT && np > 1) {
    const int64_t slot = partial_index(p, row, head, np) + part;
    float* po = p.part_o + slot * D + c * 8;
    *reinterpret_cast<f32x4*>(po) = f32x4{o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv};
    *reinterpret_cast<f32x4*>(po + 4) = f32x4{o[4] * inv, o[5] * inv, o[6] * inv, o[7] * inv};
    if (c == 0) {
      float* pml = p.part_ml + slot * 2;
      pml[0] = m;
      pml[1] = l;
    }
  } else {
    uint16_t* out = static_cast<uint16_t*>(p.out) + head_row * D + c * 8;
    u32x4 w;
    w.x = E::round(o[0] * inv) | (E::round(o[1] * inv) << 16);
    w.y = E::round(o[2] * inv) | (E::round(o[3] * inv) << 16);
    w.z = E::round(o[4] * inv) | (E::round(o[5] * inv) << 16);
    w.w = E::round(o[6] * inv) | (E::round(o[7] * inv) << 16);
    *reinterpret_cast<u32x4*>(out) = w;
  }
}

// As store_head, from a lane of the transposed P.V layout: o[t] holds elements
// 16t + 4g + i (i < 4) of head `head`; the lanes g = 0..3 of a head hold all of it.
template <int D, bool BF16, bool SPLIT>
__device__ __forceinline__ void store_head_t(const AttnParams& p, int row, int part, int np, int head, int g,
                                             const f32x4 (&o)[D / 16], float m, float l) {
  using E = Elem<BF16>;
  const float inv = (l > 0.f ? 1.0f / l : 0.f) * p.v_scale;  // exact at v_scale 1
  const int64_t head_row = (int64_t)row * p.num_heads + head;
  if (SPLIT && np > 1) {
    const int64_t slot = partial_index(p, row, head, np) + part;
    float* po = p.part_o + slot * D + 4 * g;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) *reinterpret_cast<f32x4*>(po + 16 * t) = o[t] * inv;
    if (g == 0) {
      float* pml = p.part_ml + slot * 2;
      pml[0] = m;
      pml[1] = l;
    }
  } else {
    uint16_t* out = static_cast<uint16_t*>(p.out) + head_row * D + 4 * g;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      const f32x4 v = o[t] * inv;
      *reinterpret_cast<u32x2*>(out + 16 * t) =
          u32x2{E::round(v.x) | (E::round(v.y) << 16), E::round(v.z) | (E::round(v.w) << 16)};
    }
  }
}

// Merge partitions [0, np) of heads [head_lo, head_hi) of `row` and round into
// out: o = sum_i w_i o_i / sum_i w_i with w_i = l_i 2^(m_i - max m), folded in
// partition order (so the result does not depend on which workgroup merges).
// Thread t owns items t, t + threads, ... (an item = one head's 4 elements), at
// most IPT of them, and loads partition i of all its items before folding them,
// two partitions at a time, so the loads of one thread overlap.
template <int D, int IPT, bool BF16>
__device__ __forceinline__ void merge_partitions(const AttnParams& p, int row, int np, int head_lo, int head_hi,
                                                 int tid, int threads) {
  using E = Elem<BF16>;
  constexpr int QUADS = D / 4;
  const int items = (head_hi - head_lo) * QUADS;
  const float* ml[IPT];
  const f32x4* po[IPT];
  float m[IPT], l[IPT];
  f32x4 acc[IPT];
#pragma unroll
  for (int k = 0; k < IPT; ++k) {
    const int it = min(tid + k * threads, items - 1);  // spare slots repeat the last item, unstored
    const int64_t first = partial_index(p, row, head_lo + it / QUADS, np);
    ml[k] = p.part_ml + first * 2;
    po[k] = reinterpret_cast<const f32x4*>(p.part_o + first * D) + it % QUADS;
    m[k] = kNoScore;
    l[k] = 0.f;
    acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  auto fold = [&](int k, float mi, float wi, f32x4 v) {
    const float mn = fmaxf(m[k], mi);
    const float a = fast_exp2(m[k] - mn);
    const float b = wi * fast_exp2(mi - mn);
    l[k] = l[k] * a + b;
    acc[k] = acc[k] * a + v * b;
    m[k] = mn;
  };
  int i = 0;
  for (; i + 2 <= np; i += 2) {
    float2 s0[IPT], s1[IPT];
    f32x4 v0[IPT], v1[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
      s0[k] = reinterpret_cast<const float2*>(ml[k])[i];
      s1[k] = reinterpret_cast<const float2*>(ml[k])[i + 1];
      v0[k] = po[k][(int64_t)i * QUADS];
      v1[k] = po[k][(int64_t)(i + 1) * QUADS];
    }
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
      fold(k, s0[k].x, s0[k].y, v0[k]);
      fold(k, s1[k].x, s1[k].y, v1[k]);
    }
  }
  if (i < np) {
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
      const float2 s0 = reinterpret_cast<const float2*>(ml[k])[i];
      fold(k, s0.x, s0.y, po[k][(int64_t)i * QUADS]);
    }
  }
#pragma unroll
  for (int k = 0; k < IPT; ++k) {
    const int it = tid + k * threads;
    if (it >= items) break;
    const float inv = l[k] > 0.f ? 1.0f / l[k] : 0.f;
    const int64_t head_row = (int64_t)row * p.num_heads + head_lo + it / QUADS;
    uint32_t* o32 = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.out) + head_row * D) + (it % QUADS) * 2;
    o32[0] = E::round(acc[k].x * inv) | (E::round(acc[k].y * inv) << 16);
    o32[1] = E::round(acc[k].z * inv) | (E::round(acc[k].w * inv) << 16);
  }
}

// End of a v2 workgroup of the single-launch path (p.arrivals set). Every
// thread calls it after its partial stores. Each workgroup of a (row, head
// group) with tokens adds one to that pair's arrival counter once its partials
// are visible device-wide; the workgroup whose add completes the count -- the
// row's np partitions -- merges them, then returns the counter to zero for the
// next call. Nothing waits on another workgroup. `s_flag` is one int of LDS.
//
// Ordering: the barrier orders every wave's partial stores before thread 0's
// device-scope release fence, which precedes its counter add; the merging
// workgroup's acquire fence follows the add that read every other one. One
// release (an L2 write-back) per workgroup and one acquire (an L2 invalidate)
// per merge: per-thread device fences would cost far more than the merge saves.
template <int D, int GC, bool BF16>
__device__ __forceinline__ void arrive_and_merge(const AttnParams& p, int row, int group, int groups, int np,
                                                 int head_lo, int head_hi, int tid, int threads, int* s_flag) {
  __syncthreads();
  if (tid == 0) {
    uint32_t* counter = p.arrivals + (int64_t)row * groups + group;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const uint32_t before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = before + 1 == (uint32_t)np;
    if (last) {
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    *s_flag = last;
  }
  __syncthreads();
  if (!*s_flag) return;
  // A workgroup holds at most GC heads per wave, so GC * D / 4 items per 64 threads.
  merge_partitions<D, (GC * D / 4 + kWave - 1) / kWave, BF16>(p, row, np, head_lo, head_hi, tid, threads);
}

// Zero the output rows of GC heads of a padding row (v1): nothing of the cache is read.
template <int D, int GC, int THREADS>
__device__ __forceinline__ void store_zero_rows(const AttnParams& p, int row, int h0, int tid) {
  constexpr int LPT = D / 8;
  uint16_t* out = static_cast<uint16_t*>(p.out);
  for (int it = tid; it < GC * LPT; it += THREADS) {
    const int g = it / LPT, cc = it % LPT;
    *reinterpret_cast<u32x4*>(out + ((int64_t)row * p.num_heads + h0 + g) * D + cc * 8) =
        u32x4{0u, 0u, 0u, 0u};
  }
}

// Stage the block-table entries of positions [s0, s1) in LDS as element offsets
// of their blocks (block id x block stride; ids outside the pool become the
// padding block 0); returns the first staged block index. The host checks that
// every offset in the pool fits 32 bits.
__device__ __forceinline__ int stage_table(const AttnParams& p, const int32_t* tbl, uint32_t* s_tbl, int s0, int s1,
                                           int tid, int threads) {
  const int b0 = block_of(p, s0);
  const int nb = block_of(p, s1 - 1) - b0 + 1;
  __syncthreads();  // the previous segment is done with s_tbl
  for (int i = tid; i < nb; i += threads) s_tbl[i] = table_entry(p, tbl[b0 + i]);
  __syncthreads();
  return b0;
}

// The first table segment of a context, read before the row's length is known: the blocks of
// positions [t_begin, t_begin + span), cut at the table's last block (max_len), PF entries per
// thread (entries past PF x threads are read by commit_table). Issued beside the length's load,
// it takes the table's round trip off the chain that precedes the first K/V load.
template <int PF>
struct TableAhead {
  int32_t e[PF];  // block ids as read (converted at commit_table, so nothing waits for them here)
  int b0;
  int n;
};

template <int PF>
__device__ __forceinline__ void table_ahead(const AttnParams& p, const int32_t* tbl, int t_begin, int span, int tid,
                                            int threads, TableAhead<PF>& a) {
  const int tb = imin(t_begin, p.max_len);
  const int64_t end = (int64_t)tb + span;
  const int64_t last = (end < p.max_len ? end : (int64_t)p.max_len) - 1;
  a.b0 = block_of(p, tb);
  a.n = last >= tb ? block_of(p, (int)last) - a.b0 + 1 : 0;
#pragma unroll
  for (int k = 0; k < PF; ++k) {
    const int i = tid + k * threads;
    a.e[k] = i < a.n ? tbl[a.b0 + i] : 0;
  }
}

// Stage the prefetched first segment [s0, s1) (s0 the prefetch's t_begin, s1 within its span)
// in LDS, as stage_table does; returns its first block index.
template <int PF>
__device__ __forceinline__ int commit_table(const AttnParams& p, const int32_t* tbl, uint32_t* s_tbl,
                                            const TableAhead<PF>& a, int s1, int tid, int threads) {
  const int nb = block_of(p, s1 - 1) - a.b0 + 1;
#pragma unroll
  for (int k = 0; k < PF; ++k) {
    const int i = tid + k * threads;
    if (i < nb) s_tbl[i] = table_entry(p, a.e[k]);
  }
  for (int i = tid + PF * threads; i < nb; i += threads) s_tbl[i] = table_entry(p, tbl[a.b0 + i]);
  __syncthreads();
  return a.b0;
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// O^T += V^T P^T for a 16 x 16 tile over 16 tokens: v_mfma_f32_16x16x16.
template <bool BF16>
__device__ __forceinline__ f32x4 mfma_pv(u32x2 v, u32x2 w, f32x4 acc) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, v), __builtin_bit_cast(i16x4, w),
                                                     acc, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, v), __builtin_bit_cast(f16x4, w), acc,
                                                 0, 0, 0);
  }
}

// The P of the P.V MFMA as packed 16-bit weights. A bf16 weight (8 significant
// bits) is off by up to 2^-9 of itself, the size of the accuracy bar, so bf16 P
// takes two MFMAs: packed high parts and packed parts of the remainder, both by
// truncation, |w - h - l| < 2^-14 w. An fp16 weight rounded to nearest (11 bits)
// is within 2^-12 w, and one MFMA suffices: then only `hi` is set.
constexpr bool split_p(bool bf16) { return bf16; }

// Split 4 fp32 weights w (finite, >= 0) as above.
template <bool BF16>
__device__ __forceinline__ void split_weights4(const float (&w)[4], u32x2& hi, u32x2& lo) {
  uint32_t h[2], r[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float a = w[2 * i], b = w[2 * i + 1];
    if constexpr (BF16) {
      const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
      h[i] = __builtin_amdgcn_perm(ub, ua, 0x07060302u);
      const float ra = a - __uint_as_float(ua & 0xffff0000u);
      const float rb = b - __uint_as_float(ub & 0xffff0000u);
      r[i] = __builtin_amdgcn_perm(__float_as_uint(rb), __float_as_uint(ra), 0x07060302u);
    } else {
      h[i] = __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});  // v_cvt_pk_f16_f32, to nearest
      r[i] = 0u;
    }
  }
  hi = u32x2{h[0], h[1]};
  lo = u32x2{r[0], r[1]};
}

// 4 elements of a 16-lane group's rows, transposed: lane o of each group of 16
// receives element o % 4 of the 8-byte rows read by lanes o / 4, o / 4 + 4,
// o / 4 + 8 and o / 4 + 12 of its group (ds_read_b64_tr_b16, measured).
__device__ __forceinline__ u32x2 lds_read_transposed(const uint16_t* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(p)));
}

}  // namespace ayk
