// Paged-attention decode kernels for MI355X (gfx950, CDNA4, wave64).
//
// Semantics follow the reference's decode attention
// (python/ayaka/ops/backends/torch/attention.py:237-271) and its row
// convention (python/ayaka/ops/attention.py:12-30): row n attends to
// positions [0, len_n) of its request, with scores scale * q.k, softmax and the
// value sum in fp32, and the result rounded once to the output dtype.
//
// Design (bandwidth-bound GEMV over the cache, so VALU rather than MFMA):
//  * One workgroup of 4 waves per (row, key/value head[, partition]). The G
//    query heads that share a key/value head are served from the same K/V
//    loads, so every cache byte is read once per row.
//  * A token's head_dim slice (128 or 256 contiguous bytes in either layout)
//    is read by LPT = head_dim/8 lanes with one 128-bit load each, so one load
//    instruction covers TPL = 64/LPT tokens and a 16-lane group reads 256
//    contiguous bytes.
//  * q.k uses v_dot2 (bf16/fp16 pairs, fp32 accumulate) and a DPP butterfly
//    inside the LPT-lane group; no LDS on the hot path except the block table.
//  * Online softmax per lane group (running max m and sum l in the log2
//    domain); the groups of a wave are merged with cross-lane shuffles and the
//    4 waves through LDS at the end.
//  * K of the next chunk is loaded while the current chunk is computed.
//  * The v2 ("split") variant covers partition z of each row and writes the
//    normalised partial output plus (m, l) to scratch; the last workgroup of a
//    row to finish merges the partitions with the log-sum-exp identity
//    (arrive_and_merge), or a separate reduce kernel does. A row whose context
//    fits one partition is written directly, exactly as v1 writes it.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "attention_common.h"

namespace ayk {

template <int D, int GC, int NLD, bool BF16, bool SPLIT>
__global__ __launch_bounds__(kMaxWaves * kWave) void paged_attention_kernel(const AttnParams p) {
  using E = Elem<BF16>;
  constexpr int LPT = pieces_per_position(D);  // lanes per token (8 elements = 16 bytes each)
  constexpr int TPL = positions_per_load(D);   // tokens per load instruction
  constexpr int CH = TPL * NLD;      // tokens per chunk

  __shared__ uint32_t s_tbl[kTableCap];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int threads = blockDim.x;
  const int waves = threads / kWave;
  const int groups = (p.num_virtual_heads + waves - 1) / waves;
  const WgCoord wg = wg_coord(p, groups, SPLIT);
  if (wg.row < 0) return;  // past the staged work items (uniform per workgroup)
  const int row = wg.row;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  // Wave w serves "virtual head" group * waves + w: a key/value head, or a chunk
  // of GC of its query heads when the group is split.
  const int vh = wg.group * waves + wave;
  const bool active = vh < p.num_virtual_heads;
  const int kvh = vh / p.head_chunks;
  const int h0 = kvh * p.group + (vh % p.head_chunks) * GC;
  const int r = lane / LPT;
  const int c = lane % LPT;

  const int psize = SPLIT ? wg.psize : 0;
  // positions per staged table segment: at most kTableCap blocks, whatever s0's offset
  const int seg_len = segment_positions(p, CH);
  // the row's request, then its first table segment (known from the partition alone) and its
  // length together
  const int req = row_request(p, row);
  const int32_t* tbl = p.block_table + (int64_t)req * p.table_stride;
  TableAhead<2> ahead;
  table_ahead(p, tbl, SPLIT ? wg.part * psize : 0, SPLIT ? imin(psize, seg_len) : seg_len, tid, threads, ahead);
  const int len = row_length(p, row, req);
  int t_begin = 0, t_end = len;
  const int np = SPLIT ? (len > 0 ? (len - 1) / psize + 1 : 0) : 1;  // partitions with tokens
  if constexpr (SPLIT) {
    t_begin = wg.part * psize;
    t_end = min(len, t_begin + psize);
    if (t_begin >= t_end) {  // only partitions that hold tokens are merged
      if (len == 0 && wg.part == 0 && active) store_zero_rows<D, GC, kWave>(p, row, h0, lane);  // a padding row
      return;
    }
  } else if (len == 0) {
    if (active) store_zero_rows<D, GC, kWave>(p, row, h0, lane);
    return;
  }

  // This lane's 8 elements of each of the GC query heads, kept packed for v_dot2.
  uint32_t qw[GC][4];
  if (active) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p.q + ((int64_t)row * p.num_heads + h0 + g) * D + c * 8);
      qw[g][0] = v.x; qw[g][1] = v.y; qw[g][2] = v.z; qw[g][3] = v.w;
    }
  }

  float m[GC], l[GC], o[GC][8];
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    m[g] = kNoScore;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  }

  const uint32_t token_stride = (uint32_t)p.token_stride;
  const float scale_log2 = p.scale_log2;
  const uint16_t* kbase = p.k_cache + (int64_t)kvh * p.head_stride + c * 8;
  const uint16_t* vbase = p.v_cache + (int64_t)kvh * p.head_stride + c * 8;

  for (int s0 = t_begin; s0 < t_end; s0 += seg_len) {
    const int s1 = min(t_end, s0 + seg_len);
    const int b0 = s0 == t_begin ? commit_table(p, tbl, s_tbl, ahead, s1, tid, threads)
                                 : stage_table(p, tbl, s_tbl, s0, s1, tid, threads);
    if (!active) continue;
    const int nch = (s1 - s0 + CH - 1) / CH;

    // Element offsets of this lane's NLD tokens of chunk ci (past-the-end tokens
    // are clamped to the last one and masked later).
    auto offsets = [&](int ci, uint32_t(&dst)[NLD]) {
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
        dst[j] = kv_offset(p, s_tbl, b0, chunk_position(s0, s1, ci, CH, j, TPL, r), token_stride);
      }
    };

    // Fold one chunk of keys and values into the running state.
    auto consume = [&](int ci, const u32x4(&kc)[NLD], const u32x4(&vc)[NLD]) {
      const int tb = s0 + ci * CH;
      const bool tail = tb + CH > s1;
      float s[NLD][GC];
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          float a = E::dot2(qw[g][0], kc[j].x, 0.f);
          a = E::dot2(qw[g][1], kc[j].y, a);
          a = E::dot2(qw[g][2], kc[j].z, a);
          s[j][g] = E::dot2(qw[g][3], kc[j].w, a);
        }
      }
      // Butterfly over the LPT lanes of each token, one stage at a time across all
      // NLD x GC partial sums, so consecutive DPP reads never wait on each other.
#pragma unroll
      for (int j = 0; j < NLD; ++j)
#pragma unroll
        for (int g = 0; g < GC; ++g) s[j][g] += dpp<0xB1>(s[j][g]);  // lane ^ 1
#pragma unroll
      for (int j = 0; j < NLD; ++j)
#pragma unroll
        for (int g = 0; g < GC; ++g) s[j][g] += dpp<0x4E>(s[j][g]);  // lane ^ 2
#pragma unroll
      for (int j = 0; j < NLD; ++j)
#pragma unroll
        for (int g = 0; g < GC; ++g) s[j][g] += dpp<0x141>(s[j][g]);  // other quad of 8
      if constexpr (LPT >= 16) {
#pragma unroll
        for (int j = 0; j < NLD; ++j)
#pragma unroll
          for (int g = 0; g < GC; ++g) s[j][g] += dpp<0x140>(s[j][g]);  // other 8 of 16
      }
      if constexpr (LPT >= 32) {
#pragma unroll
        for (int j = 0; j < NLD; ++j)
#pragma unroll
          for (int g = 0; g < GC; ++g) s[j][g] += __shfl_xor(s[j][g], 16);
      }
#pragma unroll
      for (int j = 0; j < NLD; ++j)
#pragma unroll
        for (int g = 0; g < GC; ++g) s[j][g] *= scale_log2;
      if (tail) {
#pragma unroll
        for (int j = 0; j < NLD; ++j)
          if (tb + j * TPL + r >= s1) {
#pragma unroll
            for (int g = 0; g < GC; ++g) s[j][g] = -INFINITY;
          }
      }
      // Online softmax with a lazily raised max: the accumulators are rescaled
      // only when some lane's chunk max exceeds its running max by the slack.
      float mx[GC];
      bool grow = false;
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        mx[g] = s[0][g];
#pragma unroll
        for (int j = 1; j < NLD; ++j) mx[g] = fmaxf(mx[g], s[j][g]);
        grow |= mx[g] > m[g] + kRescaleSlack;
      }
      if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          const float mn = fmaxf(m[g], mx[g]);
          const float alpha = fast_exp2(m[g] - mn);
          l[g] *= alpha;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
          m[g] = mn;
        }
      }
#pragma unroll
      for (int g = 0; g < GC; ++g) {
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
          s[j][g] = fast_exp2(s[j][g] - m[g]);
          l[g] += s[j][g];
        }
      }
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
        float vf[8];
        vf[0] = E::lo(vc[j].x); vf[1] = E::hi(vc[j].x);
        vf[2] = E::lo(vc[j].y); vf[3] = E::hi(vc[j].y);
        vf[4] = E::lo(vc[j].z); vf[5] = E::hi(vc[j].z);
        vf[6] = E::lo(vc[j].w); vf[7] = E::hi(vc[j].w);
        if (tail && tb + j * TPL + r >= s1) {
          // A slot past the context may hold anything, NaN included, and 0 * NaN is NaN.
#pragma unroll
          for (int e = 0; e < 8; ++e) vf[e] = 0.f;
        }
#pragma unroll
        for (int g = 0; g < GC; ++g) {
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] = fmaf(s[j][g], vf[e], o[g][e]);
        }
      }
    };

    // Two register sets, used alternately: while one chunk is folded in, the
    // keys of the next chunk are already in flight (unrolled twice so no copies).
    uint32_t offA[NLD], offB[NLD];
    u32x4 kA[NLD], kB[NLD], vc[NLD];
    int ci = 0;
    offsets(0, offA);
#pragma unroll
    for (int j = 0; j < NLD; ++j) kA[j] = stream_load(kbase + offA[j]);
    while (ci < nch) {
#pragma unroll
      for (int j = 0; j < NLD; ++j) vc[j] = stream_load(vbase + offA[j]);
      if (ci + 1 < nch) {
        offsets(ci + 1, offB);
#pragma unroll
        for (int j = 0; j < NLD; ++j) kB[j] = stream_load(kbase + offB[j]);
      }
      consume(ci, kA, vc);
      if (++ci >= nch) break;
#pragma unroll
      for (int j = 0; j < NLD; ++j) vc[j] = stream_load(vbase + offB[j]);
      if (ci + 1 < nch) {
        offsets(ci + 1, offA);
#pragma unroll
        for (int j = 0; j < NLD; ++j) kA[j] = stream_load(kbase + offA[j]);
      }
      consume(ci, kB, vc);
      ++ci;
    }
  }
  if (active) {
    // Merge the TPL lane groups of this wave (butterfly: every group ends with the merged state).
#pragma unroll
    for (int st = LPT; st < kWave; st <<= 1) {
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        const float m2 = __shfl_xor(m[g], st);
        const float l2 = __shfl_xor(l[g], st);
        const float mn = fmaxf(m[g], m2);
        const float a = fast_exp2(m[g] - mn);
        const float b = fast_exp2(m2 - mn);
        l[g] = l[g] * a + l2 * b;
        m[g] = mn;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = o[g][e] * a + __shfl_xor(o[g][e], st) * b;
      }
    }
    if (r == 0) {
#pragma unroll
      for (int g = 0; g < GC; ++g)
        store_head<D, BF16, SPLIT>(p, row, wg.part, np, h0 + g, c, o[g], m[g], l[g]);
    }
  }
  if constexpr (SPLIT) {
    if (np > 1 && p.arrivals) {
      const int vh_lo = wg.group * waves;
      const int vh_hi = min(p.num_virtual_heads, vh_lo + waves);
      arrive_and_merge<D, GC, BF16>(p, row, wg.group, groups, np, vh_lo * GC, vh_hi * GC, tid, threads, &s_last);
    }
  }
}

// Merge the partitions of (row, head) pairs: o = sum_p w_p o_p / sum_p w_p with
// w_p = l_p * 2^(m_p - max m). A workgroup serves HEADS = 256 / (S * D/4)
// consecutive (row, head) pairs, S * D/4 threads each: thread t of a pair owns 4
// elements (t % (D/4)) of every S-th partition from t / (D/4) on and merges them
// online (its own running max), so its partial loads are independent; the S
// partial merges then meet in LDS with the same log-sum-exp rule. The host
// takes S = 1 for up to 4 partitions per row, or up to 16 when the grid still
// gives every compute unit a workgroup (one workgroup then merges 8 heads at
// D 128), and more slots for long rows, whose serial folds would otherwise be
// long. A row with
// one partition was written by the partition kernel, so v2 with a single
// partition rounds exactly the value v1 rounds; a row without context gets zeros.
constexpr int kReduceThreads = 256;

// F32: an fp32 model's merge, its output written in fp32 (BF16 then unused).
template <int D, bool BF16, int S, bool F32 = false>
__global__ __launch_bounds__(kReduceThreads) void partition_reduce_kernel(const AttnParams p) {
  using E = Elem<BF16>;
  constexpr int QUADS = D / 4;                // float4 groups of a row
  constexpr int HEADS = kReduceThreads / (S * QUADS);
  static_assert(HEADS >= 1 && HEADS * S * QUADS == kReduceThreads, "reduce shape");
  __shared__ f32x4 s_acc[HEADS][S][QUADS];
  __shared__ float s_m[HEADS][S];
  __shared__ float s_l[HEADS][S];

  const int tid = threadIdx.x;
  const int hl = tid / (S * QUADS);
  const int quad = tid % QUADS;
  const int slot = (tid / QUADS) % S;
  const int64_t pair = (int64_t)blockIdx.x * HEADS + hl;  // (row, head) over n_rows x num_heads
  const bool valid = pair < (int64_t)p.n_rows * p.num_heads;
  // 32-bit division: the host refuses n_rows x num_heads above INT32_MAX
  const int pair32 = valid ? (int)pair : 0;
  const int row = pair32 / p.num_heads;
  const int head = pair32 - row * p.num_heads;
  // the row's first partial slot of a staged launch, read with the row's context
  const int staged_first = *(p.staged ? p.staged + 2 + row : p.kv_lengths);
  int req, len;
  row_context(p, row, req, len);
  const int np = valid ? (len > 0 ? (len - 1) / partition_size_of(p) + 1 : 0) : 1;
  // partial_index, with the staged slot read above
  const int64_t first = p.staged ? (int64_t)staged_first * p.num_heads + (int64_t)head * np
                                 : ((int64_t)row * p.num_heads + head) * p.max_partitions;
  const float* ml = p.part_ml + first * 2;
  const f32x4* po = reinterpret_cast<const f32x4*>(p.part_o + first * D);

  float m = kNoScore, l = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int nfold = np > 1 ? np : 0;  // rows of one partition (or none) fold nothing
  auto fold = [&](float mi, float wi, f32x4 v, bool real) {
    const float mn = real ? fmaxf(m, mi) : m;
    const float a = fast_exp2(m - mn);
    const float b = real ? wi * fast_exp2(mi - mn) : 0.f;
    l = l * a + b;
    acc = acc * a + v * b;
    m = mn;
  };
  if constexpr (S == 1) {
    // One slot: the thread folds its pair's partitions one by one (with one slot the
    // grid is wide and the rows hold few partitions; batched loads measured no faster).
#pragma unroll 4
    for (int i = 0; i < nfold; ++i) fold(ml[2 * i], ml[2 * i + 1], po[(int64_t)i * QUADS + quad], true);
  } else {
    // 8 partitions per thread per batch, all loaded before the first is folded (indices
    // past the last partition read the last one, folded with weight 0), so a batch costs
    // one memory round trip, not one per partition; the fold order is the thread's
    // partitions in order, as one at a time.
    constexpr int B = 8;
    for (int base = 0; base < nfold; base += B * S) {
      float mi[B], wi[B];
      f32x4 vi[B];
#pragma unroll
      for (int k = 0; k < B; ++k) {
        const int i = min(base + slot + k * S, nfold - 1);
        mi[k] = ml[2 * i];
        wi[k] = ml[2 * i + 1];
        vi[k] = po[(int64_t)i * QUADS + quad];
      }
#pragma unroll
      for (int k = 0; k < B; ++k) fold(mi[k], wi[k], vi[k], base + slot + k * S < nfold);
    }
  }
  if constexpr (S > 1) {
    s_acc[hl][slot][quad] = acc;
    if (quad == 0) {
      s_m[hl][slot] = m;
      s_l[hl][slot] = l;
    }
    __syncthreads();
  }
  if (slot != 0 || np == 1) return;
  float mn = m, L = l;
  f32x4 total = acc;
  if constexpr (S > 1) {
    mn = s_m[hl][0];
#pragma unroll
    for (int k = 1; k < S; ++k) mn = fmaxf(mn, s_m[hl][k]);
    total = f32x4{0.f, 0.f, 0.f, 0.f};
    L = 0.f;
#pragma unroll
    for (int k = 0; k < S; ++k) {
      const float w = fast_exp2(s_m[hl][k] - mn);
      L += s_l[hl][k] * w;
      total += s_acc[hl][k][quad] * w;
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;  // np == 0: zeros
  if constexpr (F32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + pair * D + quad * 4) = total * inv;
  } else {
    uint32_t* o32 = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.out) + pair * D) + quad * 2;
    o32[0] = E::round(total.x * inv) | (E::round(total.y * inv) << 16);
    o32[1] = E::round(total.z * inv) | (E::round(total.w * inv) << 16);
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch.

template <int D, int GC, bool BF16>
static hipError_t launch_dpp_typed(const AttnParams& p, bool split, hipStream_t stream) {
  // Two loads per token slot per chunk: 8 tokens (D 128), 16 (D 64) or 4 (D 256) per
  // chunk keeps a group of 4 under 128 VGPRs, so two 8-wave workgroups share a CU.
  constexpr int NLD = dpp_loads_per_chunk();
  // One wave per virtual head, up to kMaxWaves per workgroup.
  const int waves = p.num_virtual_heads < kMaxWaves ? p.num_virtual_heads : kMaxWaves;
  const int groups = (p.num_virtual_heads + waves - 1) / waves;
  const int64_t items = (split && p.work) ? p.n_work : (int64_t)p.n_rows * (split ? p.max_partitions : 1);
  const dim3 grid((unsigned)(items * groups)), block(waves * kWave);
  if (split)
    hipLaunchKernelGGL((paged_attention_kernel<D, GC, NLD, BF16, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((paged_attention_kernel<D, GC, NLD, BF16, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <int D, bool BF16>
static hipError_t launch_dpp_gc(const AttnParams& p, int gc, bool split, hipStream_t stream) {
  switch (gc) {
    case 1: return launch_dpp_typed<D, 1, BF16>(p, split, stream);
    case 2: return launch_dpp_typed<D, 2, BF16>(p, split, stream);
    case 3: return launch_dpp_typed<D, 3, BF16>(p, split, stream);
    case 4: return launch_dpp_typed<D, 4, BF16>(p, split, stream);
    case 5: return launch_dpp_typed<D, 5, BF16>(p, split, stream);
    case 6: return launch_dpp_typed<D, 6, BF16>(p, split, stream);
    case 7: return launch_dpp_typed<D, 7, BF16>(p, split, stream);
    case 8: return launch_dpp_typed<D, 8, BF16>(p, split, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attention_dpp(const AttnParams& p, int head_dim, int gc, bool bf16, bool split, int waves,
                                hipStream_t stream) {
  (void)waves;  // one workgroup shape (4 waves) for this kernel
  switch (head_dim) {
    case 64: return bf16 ? launch_dpp_gc<64, true>(p, gc, split, stream)
                         : launch_dpp_gc<64, false>(p, gc, split, stream);
    case 128: return bf16 ? launch_dpp_gc<128, true>(p, gc, split, stream)
                          : launch_dpp_gc<128, false>(p, gc, split, stream);
    case 256: return bf16 ? launch_dpp_gc<256, true>(p, gc, split, stream)
                          : launch_dpp_gc<256, false>(p, gc, split, stream);
    default: return hipErrorInvalidValue;
  }
}

// Merge of the multi-row kernel's partitions: one workgroup per row, all its
// query heads (a row's heads lie next to each other in the partials), so a step
// of many rows launches one workgroup per row rather than per (row, head). Rows
// with one partition were written by the partition kernel and rows of padding
// requests were zeroed by it; both return at once.
template <int D, bool BF16>
__global__ __launch_bounds__(kReduceThreads) void row_reduce_kernel(const AttnParams p) {
  constexpr int IPT = 4;
  constexpr int HEADS_PER_PASS = kReduceThreads * IPT / (D / 4);
  const int row = blockIdx.x;
  int req, len;
  row_context(p, row, req, len);
  const int np = len > 0 ? (len - 1) / p.partition_size + 1 : 0;
  if (np <= 1) return;
  for (int h0 = 0; h0 < p.num_heads; h0 += HEADS_PER_PASS)
    merge_partitions<D, IPT, BF16>(p, row, np, h0, min(p.num_heads, h0 + HEADS_PER_PASS), threadIdx.x,
                                   kReduceThreads);
}

hipError_t launch_row_reduce(const AttnParams& p, int head_dim, bool bf16, hipStream_t stream) {
  const dim3 grid((unsigned)p.n_rows), block(kReduceThreads);
  switch (head_dim) {
    case 64:
      if (bf16) hipLaunchKernelGGL((row_reduce_kernel<64, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((row_reduce_kernel<64, false>), grid, block, 0, stream, p);
      break;
    case 128:
      if (bf16) hipLaunchKernelGGL((row_reduce_kernel<128, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((row_reduce_kernel<128, false>), grid, block, 0, stream, p);
      break;
    case 256:
      if (bf16) hipLaunchKernelGGL((row_reduce_kernel<256, true>), grid, block, 0, stream, p);
      else hipLaunchKernelGGL((row_reduce_kernel<256, false>), grid, block, 0, stream, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int D, bool BF16, bool F32 = false>
static hipError_t launch_reduce_typed(const AttnParams& p, int compute_units, hipStream_t stream) {
  // Partition slots per (row, head): one for up to 4 partitions per row, and up to 16 when
  // one slot still gives every compute unit a workgroup (many pairs, most of whose rows often
  // hold one partition and merge nothing: a ragged batch's grid of 2-pair workgroups spent
  // ~4 us more in residency rounds); then 4, or as many as one workgroup holds for a single
  // head when 4 would leave compute units without a workgroup (few rows of many partitions:
  // 8 rows x 32 heads over 32K). A staged launch sizes max_partitions for its smallest
  // partition size while its steps mostly run far fewer, so 4 slots serve it unless the grid
  // is small.
  constexpr int QUADS = D / 4;
  constexpr int S_MAX = kReduceThreads / QUADS;
  constexpr int S4 = S_MAX < 4 ? S_MAX : 4;
  const int64_t pairs = (int64_t)p.n_rows * p.num_heads;
  const int64_t groups1 = (pairs + S_MAX - 1) / S_MAX;
  const int64_t groups4 = (pairs + S_MAX / S4 - 1) / (S_MAX / S4);
  const bool one_slot = p.max_partitions <= 4 || (p.max_partitions <= 16 && groups1 >= compute_units);
  const int s = one_slot ? 1 : (p.max_partitions <= 16 || groups4 >= compute_units) ? S4 : S_MAX;
  const dim3 block(kReduceThreads);
  auto grid = [&](int heads) { return dim3((unsigned)((pairs + heads - 1) / heads)); };
  if (s == 1) hipLaunchKernelGGL((partition_reduce_kernel<D, BF16, 1, F32>), grid(S_MAX), block, 0, stream, p);
  else if (s == S4)
    hipLaunchKernelGGL((partition_reduce_kernel<D, BF16, S4, F32>), grid(S_MAX / S4), block, 0, stream, p);
  else hipLaunchKernelGGL((partition_reduce_kernel<D, BF16, S_MAX, F32>), grid(1), block, 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_partition_reduce_f32(const AttnParams& p, int head_dim, int compute_units, hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_reduce_typed<64, false, true>(p, compute_units, stream);
    case 128: return launch_reduce_typed<128, false, true>(p, compute_units, stream);
    case 256: return launch_reduce_typed<256, false, true>(p, compute_units, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_partition_reduce(const AttnParams& p, int head_dim, bool bf16, int compute_units,
                                   hipStream_t stream) {
  const int cu = compute_units;
  switch (head_dim) {
    case 64: return bf16 ? launch_reduce_typed<64, true>(p, cu, stream) : launch_reduce_typed<64, false>(p, cu, stream);
    case 128:
      return bf16 ? launch_reduce_typed<128, true>(p, cu, stream) : launch_reduce_typed<128, false>(p, cu, stream);
    case 256:
      return bf16 ? launch_reduce_typed<256, true>(p, cu, stream) : launch_reduce_typed<256, false>(p, cu, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ayk
