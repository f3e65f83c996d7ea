// KV-cache write and whole-block kernels for MI355X (gfx950).
//
// reshape_and_cache follows the reference's KVCacheOps.store
// (python/ayaka/ops/backends/torch/kvcache.py:65-80): row i of k and v lands in
// slot slot_mapping[i] = block * block_size + offset, bit for bit. It is pure
// data movement, so each lane moves one 16-byte vector (8 fp16/bf16 elements)
// and consecutive lanes cover consecutive bytes of a row: in NHD a row's
// destination (one slot, all heads) is contiguous, in HND each head's slice of
// it is.
//
// The block kernels (gather / copy_blocks / zero_blocks, same file :83-115)
// move whole blocks: a block is block_size * kv_heads * head_dim contiguous
// elements in either layout.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ayaka_hip_internal.h"

namespace ayk {

template <int VEC>
struct VecOf;
template <>
struct VecOf<16> { typedef uint32_t T __attribute__((ext_vector_type(4))); };
template <>
struct VecOf<8> { typedef uint32_t T __attribute__((ext_vector_type(2))); };
template <>
struct VecOf<4> { typedef uint32_t T; };
template <>
struct VecOf<2> { typedef uint16_t T; };

template <>
struct VecOf<1> { typedef uint8_t T; };

// fp32 to an OCP fp8 e4m3 code (the float8_e4m3fn format: sign, 4 exponent bits
// with bias 7, 3 mantissa bits, no infinity, NaN = 0x7F/0xFF), rounding to
// nearest even. A magnitude that rounds above the largest finite value, 448,
// becomes NaN, as does NaN: the format has no saturation here. Below 2^-6 the
// codes are the subnormals m * 2^-9.
__device__ __forceinline__ uint32_t e4m3_code(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t mag = u & 0x7fffffffu;
  const float a = __uint_as_float(mag);
  uint32_t code;
  if (a < 0.015625f) {
    code = (uint32_t)__builtin_rintf(a * 512.0f);  // ties to even; 8 is the smallest normal, 2^-6
  } else {
    // keep 3 mantissa bits, ties to even, and move the exponent from bias 127 to bias 7
    code = ((mag + 0x7ffffu + ((mag >> 20) & 1u)) >> 20) - (120u << 3);
    if (code > 0x7eu) code = 0x7fu;  // above 448, infinity or NaN
  }
  return code | sign;
}

template <bool BF16>
__device__ __forceinline__ float widen(uint32_t h) {
  if constexpr (BF16) return __uint_as_float(h << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// KV write into fp8 caches: as reshape_and_cache, but each lane reads EPL
// consecutive 16-bit elements of a row and writes their EPL codes, each element
// first multiplied by its tensor's inverse scale (one fp32 rounding; 1 leaves it as is).
template <int EPL, bool BF16>
__global__ __launch_bounds__(256) void reshape_and_cache_e4m3_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint8_t* __restrict__ k_cache,
    uint8_t* __restrict__ v_cache, const int64_t* __restrict__ slot_mapping, int64_t total_groups,
    int32_t groups_per_row, int32_t groups_per_head, int64_t num_slots, int32_t block_size, int32_t num_kv_heads,
    int32_t head_dim, int32_t hnd, float k_inv, float v_inv) {
  typedef typename VecOf<2 * EPL>::T In;
  typedef typename VecOf<EPL>::T Out;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total_groups) return;
  const int64_t row = idx / groups_per_row;
  const int32_t gi = (int32_t)(idx - row * groups_per_row);
  const int64_t slot = slot_mapping[row];
  if (slot < 0 || slot >= num_slots) return;  // outside the pool: dropped, never written
  const int64_t row_elems = (int64_t)groups_per_row * EPL;
  const int64_t src = row * row_elems + (int64_t)gi * EPL;
  int64_t dst;
  if (!hnd) {
    dst = slot * row_elems + (int64_t)gi * EPL;
  } else {
    const int64_t blk = slot / block_size;
    const int64_t off = slot - blk * block_size;
    const int32_t h = gi / groups_per_head;
    const int32_t w = gi - h * groups_per_head;
    dst = ((blk * num_kv_heads + h) * block_size + off) * head_dim + (int64_t)w * EPL;
  }
  const uint16_t* srcs[2] = {k + src, v + src};
  uint8_t* dsts[2] = {k_cache + dst, v_cache + dst};
  const float invs[2] = {k_inv, v_inv};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const In in = *reinterpret_cast<const In*>(srcs[t]);
    uint16_t h[EPL];
    __builtin_memcpy(h, &in, sizeof(In));
    uint8_t c[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) c[e] = (uint8_t)e4m3_code(widen<BF16>(h[e]) * invs[t]);  // exact at 1
    Out out;
    __builtin_memcpy(&out, c, sizeof(Out));
    *reinterpret_cast<Out*>(dsts[t]) = out;
  }
}

hipError_t launch_reshape_and_cache_e4m3(const void* k, const void* v, void* k_cache, void* v_cache,
                                         const int64_t* slot_mapping, int64_t n_rows, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t num_blocks, int32_t block_size, bool hnd,
                                         bool bf16, float k_inv, float v_inv, hipStream_t stream) {
  const int epl = (head_dim % 8 == 0) ? 8 : (head_dim % 4 == 0) ? 4 : (head_dim % 2 == 0) ? 2 : 1;
  const int32_t groups_per_head = head_dim / epl;
  const int32_t groups_per_row = groups_per_head * num_kv_heads;
  const int64_t total = n_rows * groups_per_row;
  if (total == 0) return hipSuccess;
  const int64_t num_slots = (int64_t)num_blocks * block_size;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  const uint16_t* kb = static_cast<const uint16_t*>(k);
  const uint16_t* vb = static_cast<const uint16_t*>(v);
  uint8_t* kc = static_cast<uint8_t*>(k_cache);
  uint8_t* vc = static_cast<uint8_t*>(v_cache);
#define AYK_E4M3_STORE(E)                                                                               \
  do {                                                                                                  \
    if (bf16)                                                                                           \
      hipLaunchKernelGGL((reshape_and_cache_e4m3_kernel<E, true>), grid, block, 0, stream, kb, vb, kc, vc, \
                         slot_mapping, total, groups_per_row, groups_per_head, num_slots, block_size,      \
                         num_kv_heads, head_dim, (int32_t)hnd, k_inv, v_inv);                           \
    else                                                                                                \
      hipLaunchKernelGGL((reshape_and_cache_e4m3_kernel<E, false>), grid, block, 0, stream, kb, vb, kc, vc, \
                         slot_mapping, total, groups_per_row, groups_per_head, num_slots, block_size,      \
                         num_kv_heads, head_dim, (int32_t)hnd, k_inv, v_inv);                           \
  } while (0)
  switch (epl) {
    case 8: AYK_E4M3_STORE(8); break;
    case 4: AYK_E4M3_STORE(4); break;
    case 2: AYK_E4M3_STORE(2); break;
    default: AYK_E4M3_STORE(1); break;
  }
#undef AYK_E4M3_STORE
  return hipGetLastError();
}

template <int VEC>
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(
    const uint8_t* __restrict__ k, const uint8_t* __restrict__ v, uint8_t* __restrict__ k_cache,
    uint8_t* __restrict__ v_cache, const int64_t* __restrict__ slot_mapping, int64_t total_vecs,
    int32_t vecs_per_row, int32_t vecs_per_head, int64_t num_slots, int32_t block_size,
    int32_t num_kv_heads, int32_t head_bytes, int32_t hnd) {
  typedef typename VecOf<VEC>::T V;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total_vecs) return;
  const int64_t row = idx / vecs_per_row;
  const int32_t vi = (int32_t)(idx - row * vecs_per_row);
  const int64_t slot = slot_mapping[row];
  if (slot < 0 || slot >= num_slots) return;  // outside the pool: dropped, never written
  const int64_t row_bytes = (int64_t)vecs_per_row * VEC;
  const int64_t src = row * row_bytes + (int64_t)vi * VEC;
  int64_t dst;
  if (!hnd) {
    dst = slot * row_bytes + (int64_t)vi * VEC;
  } else {
    const int64_t blk = slot / block_size;
    const int64_t off = slot - blk * block_size;
    const int32_t h = vi / vecs_per_head;
    const int32_t w = vi - h * vecs_per_head;
    dst = ((blk * num_kv_heads + h) * block_size + off) * head_bytes + (int64_t)w * VEC;
  }
  *reinterpret_cast<V*>(k_cache + dst) = *reinterpret_cast<const V*>(k + src);
  *reinterpret_cast<V*>(v_cache + dst) = *reinterpret_cast<const V*>(v + src);
}

hipError_t launch_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                                    const int64_t* slot_mapping, int64_t n_rows, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t num_blocks, int32_t block_size,
                                    bool hnd, int32_t elem_bytes, hipStream_t stream) {
  const int32_t head_bytes = head_dim * elem_bytes;
  const int vec = (head_bytes % 16 == 0) ? 16 : (head_bytes % 8 == 0) ? 8
                  : (head_bytes % 4 == 0) ? 4 : 2;
  const int32_t vecs_per_head = head_bytes / vec;
  const int32_t vecs_per_row = vecs_per_head * num_kv_heads;
  const int64_t total = n_rows * vecs_per_row;
  if (total == 0) return hipSuccess;
  const int64_t num_slots = (int64_t)num_blocks * block_size;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  const uint8_t* kb = static_cast<const uint8_t*>(k);
  const uint8_t* vb = static_cast<const uint8_t*>(v);
  uint8_t* kc = static_cast<uint8_t*>(k_cache);
  uint8_t* vc = static_cast<uint8_t*>(v_cache);
  switch (vec) {
    case 16:
      hipLaunchKernelGGL(reshape_and_cache_kernel<16>, grid, block, 0, stream, kb, vb, kc, vc,
                         slot_mapping, total, vecs_per_row, vecs_per_head, num_slots, block_size,
                         num_kv_heads, head_bytes, (int32_t)hnd);
      break;
    case 8:
      hipLaunchKernelGGL(reshape_and_cache_kernel<8>, grid, block, 0, stream, kb, vb, kc, vc,
                         slot_mapping, total, vecs_per_row, vecs_per_head, num_slots, block_size,
                         num_kv_heads, head_bytes, (int32_t)hnd);
      break;
    case 4:
      hipLaunchKernelGGL(reshape_and_cache_kernel<4>, grid, block, 0, stream, kb, vb, kc, vc,
                         slot_mapping, total, vecs_per_row, vecs_per_head, num_slots, block_size,
                         num_kv_heads, head_bytes, (int32_t)hnd);
      break;
    default:
      hipLaunchKernelGGL(reshape_and_cache_kernel<2>, grid, block, 0, stream, kb, vb, kc, vc,
                         slot_mapping, total, vecs_per_row, vecs_per_head, num_slots, block_size,
                         num_kv_heads, head_bytes, (int32_t)hnd);
      break;
  }
  return hipGetLastError();
}

__device__ __forceinline__ int64_t read_id(const void* ids, bool ids64, int64_t i) {
  return ids64 ? static_cast<const int64_t*>(ids)[i] : (int64_t) static_cast<const int32_t*>(ids)[i];
}

// grid.x = block pair i; grid.y * 256 lanes stride over the block's vectors.
template <int VEC>
__global__ __launch_bounds__(256) void block_op_kernel(int mode, const uint8_t* __restrict__ src_k,
                                                       const uint8_t* __restrict__ src_v,
                                                       uint8_t* __restrict__ dst_k,
                                                       uint8_t* __restrict__ dst_v,
                                                       const void* src_ids, const void* dst_ids,
                                                       int32_t ids64, int32_t num_blocks,
                                                       int64_t block_bytes) {
  typedef typename VecOf<VEC>::T V;
  const int64_t i = blockIdx.x;
  int64_t src_blk = 0, dst_blk = i;
  if (mode != 2) {
    src_blk = read_id(src_ids, ids64, i);
    if (src_blk < 0 || src_blk >= num_blocks) return;
  }
  if (mode != 0) {
    dst_blk = read_id(mode == 1 ? dst_ids : src_ids, ids64, i);
    if (dst_blk < 0 || dst_blk >= num_blocks) return;
  }
  const int64_t nvec = block_bytes / VEC;
  for (int64_t j = (int64_t)blockIdx.y * blockDim.x + threadIdx.x; j < nvec;
       j += (int64_t)gridDim.y * blockDim.x) {
    V* dk = reinterpret_cast<V*>(dst_k + dst_blk * block_bytes) + j;
    V* dv = reinterpret_cast<V*>(dst_v + dst_blk * block_bytes) + j;
    // Nontemporal: each byte is moved once (C3 pool, 4096 blocks: gather 4.9 -> 6.7 TB/s,
    // copy 4.8 -> 6.2 TB/s of bytes read plus written; a plain device copy runs 5.4).
    if (mode == 2) {
      __builtin_nontemporal_store(V{}, dk);
      __builtin_nontemporal_store(V{}, dv);
    } else {
      const V a = __builtin_nontemporal_load(reinterpret_cast<const V*>(src_k + src_blk * block_bytes) + j);
      const V b = __builtin_nontemporal_load(reinterpret_cast<const V*>(src_v + src_blk * block_bytes) + j);
      __builtin_nontemporal_store(a, dk);
      __builtin_nontemporal_store(b, dv);
    }
  }
}

hipError_t launch_block_op(int mode, const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                           const void* src_ids, const void* dst_ids, bool ids64, int64_t n,
                           int32_t num_blocks, int64_t block_bytes, hipStream_t stream) {
  if (n == 0 || block_bytes == 0) return hipSuccess;
  const int vec = (block_bytes % 16 == 0) ? 16 : (block_bytes % 4 == 0) ? 4 : 2;
  const int64_t nvec = block_bytes / vec;
  const unsigned gy = (unsigned)std::min<int64_t>((nvec + 255) / 256, 64);
  const dim3 grid((unsigned)n, gy), block(256);
  const uint8_t* sk = static_cast<const uint8_t*>(src_k);
  const uint8_t* sv = static_cast<const uint8_t*>(src_v);
  uint8_t* dk = static_cast<uint8_t*>(dst_k);
  uint8_t* dv = static_cast<uint8_t*>(dst_v);
  switch (vec) {
    case 16:
      hipLaunchKernelGGL(block_op_kernel<16>, grid, block, 0, stream, mode, sk, sv, dk, dv, src_ids,
                         dst_ids, (int32_t)ids64, num_blocks, block_bytes);
      break;
    case 4:
      hipLaunchKernelGGL(block_op_kernel<4>, grid, block, 0, stream, mode, sk, sv, dk, dv, src_ids,
                         dst_ids, (int32_t)ids64, num_blocks, block_bytes);
      break;
    default:
      hipLaunchKernelGGL(block_op_kernel<2>, grid, block, 0, stream, mode, sk, sv, dk, dv, src_ids,
                         dst_ids, (int32_t)ids64, num_blocks, block_bytes);
      break;
  }
  return hipGetLastError();
}

}  // namespace ayk
