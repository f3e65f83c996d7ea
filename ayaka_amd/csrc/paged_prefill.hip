// Multi-row paged attention (prefill chunks, verify windows) on the matrix cores (gfx950).
//
// Semantics: the reference's multi-row rule (python/ayaka/ops/backends/torch/
// attention.py:209-234): the rows of a request are its last rows, row j at
// position p_j attends to positions [0, p_j] of the request's paged context,
// scores scale * q.k, softmax and P.V in fp32, the output rounded once; rows of a
// padding request (kv_lengths 0) are zero.
//
// A workgroup of 4 waves serves one tile: up to 64 (row, query head) pairs of
// one request and one key/value head -- the 64 / G consecutive rows of the
// request whose G query heads read that key/value head. Every 16-position chunk
// of keys and values is loaded once per tile, cooperatively, into LDS, and each
// wave multiplies its 16 pairs against it:
//
//  * S^T = K Q^T: one v_mfma_f32_16x16x32 tile per chunk (keys from a swizzled
//    LDS tile, 16 query pairs as the B operand). Lane l holds the scores of
//    positions 4*(l/16)+i for pair l%16, so every per-pair quantity (running
//    max, weight sum, rescale) lives in the lane's own column.
//  * O^T += V^T P^T: v_mfma_f32_16x16x16 over 16-element slices of head_dim,
//    the values read from a transposed LDS tile and P^T straight from the S^T
//    registers, split into a bf16 (or fp16) high part and the residual so the
//    product keeps fp32-level accuracy (one bf16 P would cost ~2e-3 relative).
#include "attention_common.h"

namespace ayk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kPrefillWaves = 4;
// Chunks of K/V in flight per workgroup (register ring of the cooperative loads).
constexpr int DEPTH = 4;
constexpr int kPairsPerWave = 16;
constexpr int kPairsPerTile = kPrefillWaves * kPairsPerWave;

template <bool BF16>
__device__ __forceinline__ f32x4 mfma_qk32(u32x4 k, u32x4 q, f32x4 acc) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, k), __builtin_bit_cast(bf16x8, q),
                                                   acc, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, k), __builtin_bit_cast(f16x8, q),
                                                  acc, 0, 0, 0);
}

template <bool BF16>
__device__ __forceinline__ f32x4 mfma_pv16(u32x2 v, u32x2 p, f32x4 acc) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, v), __builtin_bit_cast(i16x4, p),
                                                     acc, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, v), __builtin_bit_cast(f16x4, p), acc,
                                                 0, 0, 0);
}

// Split 4 fp32 weights into a packed 16-bit high part and the packed residual.
template <bool BF16>
__device__ __forceinline__ void split_weights(const float (&w)[4], u32x2& hi, u32x2& lo) {
  using E = Elem<BF16>;
  uint32_t h[4], r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = E::round(w[i]);
    const float back = BF16 ? __uint_as_float(h[i] << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)h[i]);
    r[i] = E::round(w[i] - back);
  }
  hi = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  lo = u32x2{r[0] | (r[1] << 16), r[2] | (r[3] << 16)};
}

template <int D, bool BF16, bool KV8>
__global__ __launch_bounds__(kPrefillWaves * kWave) void paged_prefill_kernel(const AttnParams p, const int32_t* tiles) {
  using E = Elem<BF16>;
  constexpr int THREADS = kPrefillWaves * kWave;
  constexpr int CH = 16;           // positions per chunk
  constexpr int KS = D / 32;       // q.k k-steps
  constexpr int DT = D / 16;       // 16-element slices of head_dim for P.V
  constexpr int CPT = D / 8;       // 16-byte pieces per position
  constexpr int PIECES = CH * CPT; // 16-byte pieces per chunk of K (or V)
  constexpr int VT_STRIDE = CH + 4;  // halfs per transposed value row (padded against bank conflicts)

  __shared__ int s_tbl[kTableCap];
  __shared__ u32x4 s_k[2][PIECES];
  __shared__ __attribute__((aligned(16))) uint16_t s_vt[2][D * VT_STRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int mt = lane % 16;
  const int mq = lane / 16;
  const int kvh = blockIdx.x % (p.num_heads / p.group);
  const int tile = blockIdx.x / (p.num_heads / p.group);
  const int first_row = tiles[3 * tile];
  const int n_rows = tiles[3 * tile + 1];
  const int req = tiles[3 * tile + 2];
  const int group = p.group;
  const int n_pairs = n_rows * group;

  // This lane's (row, query head) pair.
  const int pair = wave * kPairsPerWave + mt;
  const bool real_pair = pair < n_pairs;
  const int prow = first_row + (real_pair ? pair / group : 0);
  const int phead = kvh * group + (real_pair ? pair % group : 0);

  int kv_len = p.kv_lengths[req];
  kv_len = max(0, min(kv_len, p.max_len));
  const int last_pos = kv_len > 0 ? min(p.positions[first_row + n_rows - 1], kv_len - 1) : -1;
  const int my_pos = real_pair && kv_len > 0 ? min(p.positions[prow], kv_len - 1) : -1;

  if (kv_len == 0) {
    // A padding request: zero rows.
    uint16_t* out = static_cast<uint16_t*>(p.out);
    for (int i = tid; i < n_pairs * CPT; i += THREADS) {
      const int pr = i / CPT, piece = i % CPT;
      const int row = first_row + pr / group, head = kvh * group + pr % group;
      *reinterpret_cast<u32x4*>(out + ((int64_t)row * p.num_heads + head) * D + piece * 8) = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }

  // q as the B operand of S^T = K Q^T: pair mt, k-slice mq of step s.
  u32x4 qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qb[s] = real_pair ? *reinterpret_cast<const u32x4*>(p.q + ((int64_t)prow * p.num_heads + phead) * D + s * 32 +
                                                        mq * 8)
                      : u32x4{0u, 0u, 0u, 0u};

  float m = kNoScore, l = 0.f;
  f32x4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* tbl = p.block_table + (int64_t)req * p.table_stride;
  const int shift = p.bs_shift;
  const int bs_mask = (1 << shift) - 1;
  const int seg_len = (((kTableCap - 1) << shift) / CH) * CH;
  const uint32_t block_stride = (uint32_t)p.block_stride;
  const uint32_t token_stride = (uint32_t)p.token_stride;
  const float scale_log2 = p.scale_log2;
  const uint16_t* kbase = kv_at<KV8>(p.k_cache, (int64_t)kvh * p.head_stride);
  const uint16_t* vbase = kv_at<KV8>(p.v_cache, (int64_t)kvh * p.head_stride);
  auto key_slot = [](int token, int piece) { return token * CPT + (piece ^ (token & (CPT - 1))); };
  constexpr int PER_THREAD = (PIECES + THREADS - 1) / THREADS;

  const int t_end = last_pos + 1;
  for (int s0 = 0; s0 < t_end; s0 += seg_len) {
    const int s1 = min(t_end, s0 + seg_len);
    const int b0 = stage_table(p, tbl, s_tbl, s0, s1, tid, THREADS);
    const int nch = (s1 - s0 + CH - 1) / CH;

    // Cooperative chunk loads: thread tid carries pieces tid, tid + THREADS, ... of
    // every chunk. A ring of DEPTH register slots keeps DEPTH chunks in flight, so the
    // HBM latency of one chunk overlaps the compute of the DEPTH - 1 before it.
    typedef typename KvRaw<KV8>::T Raw;
    Raw kr[DEPTH][PER_THREAD], vr[DEPTH][PER_THREAD];
    auto load_chunk = [&](int ci, Raw(&kd)[PER_THREAD], Raw(&vd)[PER_THREAD]) {
#pragma unroll
      for (int u = 0; u < PER_THREAD; ++u) {
        const int piece = tid + u * THREADS;
        if (PIECES % THREADS == 0 || piece < PIECES) {
          const int t = min(s0 + ci * CH + piece / CPT, s1 - 1);
          const uint32_t blk = (uint32_t)s_tbl[(t >> shift) - b0];
          const uint32_t off = blk * block_stride + (uint32_t)(t & bs_mask) * token_stride + (piece % CPT) * 8;
          kd[u] = load_kv_raw<KV8>(kbase, off);
          vd[u] = load_kv_raw<KV8>(vbase, off);
        }
      }
    };
    auto stage_chunk = [&](int buf, const Raw(&kd)[PER_THREAD], const Raw(&vd)[PER_THREAD]) {
#pragma unroll
      for (int u = 0; u < PER_THREAD; ++u) {
        const int piece = tid + u * THREADS;
        if (PIECES % THREADS == 0 || piece < PIECES) {
          const int tok = piece / CPT, c = piece % CPT;
          s_k[buf][key_slot(tok, c)] = kv_pairs<KV8, BF16>(kd[u]);
          const u32x4 vp = kv_pairs<KV8, BF16>(vd[u]);
          const uint32_t w[4] = {vp.x, vp.y, vp.z, vp.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s_vt[buf][(c * 8 + 2 * e) * VT_STRIDE + tok] = (uint16_t)(w[e] & 0xffffu);
            s_vt[buf][(c * 8 + 2 * e + 1) * VT_STRIDE + tok] = (uint16_t)(w[e] >> 16);
          }
        }
      }
    };

    // Fold chunk ci (staged in LDS buffer buf) into every pair's running state.
    auto consume = [&](int ci, int buf) {
      const int tb = s0 + ci * CH;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = mfma_qk32<BF16>(s_k[buf][key_slot(mt, s * 4 + mq)], qb[s], acc);
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = tb + 4 * mq + i;
        sc[i] = (t <= my_pos && t < s1) ? acc[i] * scale_log2 : -INFINITY;
      }
      float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      if (__builtin_amdgcn_ballot_w64(mx > m + kRescaleSlack)) {
        const float mn = fmaxf(m, mx);
        const float alpha = fast_exp2(m - mn);
        l *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t) o[t] *= alpha;
        m = mn;
      }
      float w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[i] = fast_exp2(sc[i] - m);
        l += w[i];
      }
      u32x2 phi, plo;
      split_weights<BF16>(w, phi, plo);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const u32x2 va = *reinterpret_cast<const u32x2*>(&s_vt[buf][(t * 16 + mt) * VT_STRIDE + 4 * mq]);
        o[t] = mfma_pv16<BF16>(va, phi, o[t]);
        o[t] = mfma_pv16<BF16>(va, plo, o[t]);
      }
    };

    // Loads past the last chunk re-read it (clamped) rather than being skipped, so
    // every iteration issues the same loads and the wait before each stage can
    // leave the younger chunks in flight.
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load_chunk(min(d, nch - 1), kr[d], vr[d]);
    stage_chunk(0, kr[0], vr[0]);
    lds_barrier();
    // Iteration ci: chunk ci is in LDS buffer ci & 1, chunk ci + 1 in slot (ci + 1) % DEPTH.
    // Slot ci % DEPTH was staged one iteration ago and takes chunk ci + DEPTH.
    // The chunk count is rounded up to a multiple of DEPTH, so the unrolled body has
    // no exit and the waits stay static; the extra chunks re-read the last one and
    // their positions (>= s1) are masked, so their weights are 0 (the data is real,
    // so 0 times it is 0).
    const int nch_padded = (nch + DEPTH - 1) / DEPTH * DEPTH;
    for (int base = 0; base < nch_padded; base += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int ci = base + d;
        load_chunk(min(ci + DEPTH, nch - 1), kr[d], vr[d]);
        consume(ci, ci & 1);
        stage_chunk((ci + 1) & 1, kr[(d + 1) % DEPTH], vr[(d + 1) % DEPTH]);
        lds_barrier();
      }
    }
  }

  // The pair's weight sum over the 4 position groups; lane (mq, mt) holds
  // elements 16*t + 4*mq + i of pair mt.
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (!real_pair) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  uint16_t* out = static_cast<uint16_t*>(p.out) + ((int64_t)prow * p.num_heads + phead) * D;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    uint32_t* o32 = reinterpret_cast<uint32_t*>(out + t * 16 + 4 * mq);
    o32[0] = E::round(o[t][0] * inv) | (E::round(o[t][1] * inv) << 16);
    o32[1] = E::round(o[t][2] * inv) | (E::round(o[t][3] * inv) << 16);
  }
}

template <int D>
static hipError_t launch_prefill_d(const AttnParams& p, const int32_t* tiles, dim3 grid, bool bf16, bool kv8,
                                   hipStream_t stream) {
  const dim3 block(kPrefillWaves * kWave);
  if (kv8) {
    if (bf16) hipLaunchKernelGGL((paged_prefill_kernel<D, true, true>), grid, block, 0, stream, p, tiles);
    else hipLaunchKernelGGL((paged_prefill_kernel<D, false, true>), grid, block, 0, stream, p, tiles);
  } else {
    if (bf16) hipLaunchKernelGGL((paged_prefill_kernel<D, true, false>), grid, block, 0, stream, p, tiles);
    else hipLaunchKernelGGL((paged_prefill_kernel<D, false, false>), grid, block, 0, stream, p, tiles);
  }
  return hipGetLastError();
}

hipError_t launch_prefill(const AttnParams& p, const int32_t* tiles, int n_tiles, int head_dim, bool bf16, bool kv8,
                          hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)n_tiles * (p.num_heads / p.group)));
  switch (head_dim) {
    case 64: return launch_prefill_d<64>(p, tiles, grid, bf16, kv8, stream);
    case 128: return launch_prefill_d<128>(p, tiles, grid, bf16, kv8, stream);
    case 256: return launch_prefill_d<256>(p, tiles, grid, bf16, kv8, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ayk
