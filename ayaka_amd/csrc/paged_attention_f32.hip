// Paged-attention decode for fp32 models (fp32 q, out and caches) on MI355X (gfx950).
//
// Semantics: the reference's decode rule (python/ayaka/ops/backends/torch/attention.py:237-271)
// over fp32 caches, which its torch backend serves and flashinfer refuses
// (python/ayaka/ops/backends/flashinfer/attention.py:298-301): row n attends to positions
// [0, len_n) of its request, scores scale * q.k, softmax and the value sum in fp32, and the
// output written in fp32. Rows with a position (multi-row steps run row by row here) see
// [0, position].
//
// The path is bandwidth-bound like the 16-bit decode kernels, with twice the bytes per
// position, so it keeps their shape on the VALU: one workgroup per (row[, partition]) and group
// of up to 8 virtual heads, one wave per virtual head (a key/value head, or a chunk of up to 8 of
// its query heads). A token's head_dim row (D fp32 = 4D bytes) is read by D/4 lanes with one
// 16-byte nontemporal load each, so a load instruction covers 64 / (D/4) tokens; q.k is four FMAs
// per lane and head, summed over the token's lanes by DPP and cross-lane shuffles; each lane group
// keeps its own online softmax (log2 domain, lazily raised max) and the groups meet by shuffles at
// the end. The next chunk's keys are in flight while the current chunk is folded. v2 writes each
// partition's normalised partial and (m, l), merged by partition_reduce_kernel with fp32 output.

#include "attention_common.h"

namespace ayk {

template <int D, int GC, bool SPLIT>
__global__ __launch_bounds__(kMaxWaves * kWave) void paged_attention_f32_kernel(const AttnParams p) {
  constexpr int F = f32_floats_per_lane(GC);       // floats of a token a lane reads (4 or 8)
  constexpr int FQ = F / 4;                        // its 16-byte loads
  constexpr int LPT = f32_lanes_per_position(D, GC);  // lanes per token
  constexpr int TPL = kWave / LPT;                 // tokens per load instruction
  constexpr int NLD = f32_loads_per_chunk(GC);     // token slots per lane and chunk
  constexpr int CH = TPL * NLD;                    // tokens per chunk
  typedef f32x4 Row[FQ];

  __shared__ uint32_t s_tbl[kTableCap];

  const int tid = threadIdx.x;
  const int threads = blockDim.x;
  const int waves = threads / kWave;
  const int groups = (p.num_virtual_heads + waves - 1) / waves;
  const WgCoord wg = wg_coord(p, groups, SPLIT);
  if (wg.row < 0) return;  // past the staged work items (uniform per workgroup)
  const int row = wg.row;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int vh = wg.group * waves + wave;
  const bool active = vh < p.num_virtual_heads;
  const int kvh = vh / p.head_chunks;
  const int h0 = kvh * p.group + (vh % p.head_chunks) * GC;
  const int r = lane / LPT;
  const int c = lane % LPT;
  float* out = static_cast<float*>(p.out);

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
    t_end = imin(len, t_begin + psize);
  }
  if (t_begin >= t_end) {
    // a padding row gets zeros (from partition 0); a partition past the row's context: nothing
    if (len == 0 && wg.part == 0 && active && r == 0) {
#pragma unroll
      for (int g = 0; g < GC; ++g)
#pragma unroll
        for (int u = 0; u < FQ; ++u)
          *reinterpret_cast<f32x4*>(out + ((int64_t)row * p.num_heads + h0 + g) * D + c * F + 4 * u) =
              f32x4{0.f, 0.f, 0.f, 0.f};
    }
    return;
  }

  Row qv[GC], o[GC];
  float m[GC], l[GC];
#pragma unroll
  for (int g = 0; g < GC; ++g) {
#pragma unroll
    for (int u = 0; u < FQ; ++u) {
      qv[g][u] = active ? *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p.q) +
                                                          ((int64_t)row * p.num_heads + h0 + g) * D + c * F + 4 * u)
                        : f32x4{0.f, 0.f, 0.f, 0.f};
      o[g][u] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    m[g] = kNoScore;
    l[g] = 0.f;
  }

  const uint32_t token_stride = (uint32_t)p.token_stride;
  const float scale_log2 = p.scale_log2;
  const float* kbase = reinterpret_cast<const float*>(p.k_cache) + (int64_t)kvh * p.head_stride + c * F;
  const float* vbase = reinterpret_cast<const float*>(p.v_cache) + (int64_t)kvh * p.head_stride + c * F;

  for (int s0 = t_begin; s0 < t_end; s0 += seg_len) {
    const int s1 = imin(t_end, s0 + seg_len);
    const int b0 = s0 == t_begin ? commit_table(p, tbl, s_tbl, ahead, s1, tid, threads)
                                 : stage_table(p, tbl, s_tbl, s0, s1, tid, threads);
    if (!active) continue;
    const int nch = (s1 - s0 + CH - 1) / CH;

    auto offsets = [&](int ci, uint32_t(&dst)[NLD]) {
#pragma unroll
      for (int j = 0; j < NLD; ++j)
        dst[j] = kv_offset(p, s_tbl, b0, chunk_position(s0, s1, ci, CH, j, TPL, r), token_stride);
    };
    auto load = [](const float* base, uint32_t off, Row& dst) {
#pragma unroll
      for (int u = 0; u < FQ; ++u) dst[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(base + off) + u);
    };

    auto consume = [&](int ci, const Row(&kc)[NLD], const Row(&vc)[NLD]) {
      const int tb = s0 + ci * CH;
      const bool tail = tb + CH > s1;
      float s[NLD][GC];
#pragma unroll
      for (int j = 0; j < NLD; ++j)
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          float a = qv[g][0].x * kc[j][0].x;
          a = fmaf(qv[g][0].y, kc[j][0].y, a);
          a = fmaf(qv[g][0].z, kc[j][0].z, a);
          a = fmaf(qv[g][0].w, kc[j][0].w, a);
#pragma unroll
          for (int u = 1; u < FQ; ++u) {
            a = fmaf(qv[g][u].x, kc[j][u].x, a);
            a = fmaf(qv[g][u].y, kc[j][u].y, a);
            a = fmaf(qv[g][u].z, kc[j][u].z, a);
            a = fmaf(qv[g][u].w, kc[j][u].w, a);
          }
          s[j][g] = a;
        }
      // Sum over the token's LPT lanes, one stage at a time across all the partial sums.
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
        for (int g = 0; g < GC; ++g) s[j][g] += dpp<0x141>(s[j][g]);  // the other quad of 8
      if constexpr (LPT >= 16) {
#pragma unroll
        for (int j = 0; j < NLD; ++j)
#pragma unroll
          for (int g = 0; g < GC; ++g) s[j][g] += dpp<0x140>(s[j][g]);  // the other 8 of 16
      }
      if constexpr (LPT >= 32) {
#pragma unroll
        for (int j = 0; j < NLD; ++j)
#pragma unroll
          for (int g = 0; g < GC; ++g) s[j][g] += __shfl_xor(s[j][g], 16);
      }
      if constexpr (LPT >= 64) {
#pragma unroll
        for (int j = 0; j < NLD; ++j)
#pragma unroll
          for (int g = 0; g < GC; ++g) s[j][g] += __shfl_xor(s[j][g], 32);
      }
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
        const bool past = tail && tb + j * TPL + r >= s1;
#pragma unroll
        for (int g = 0; g < GC; ++g) s[j][g] = past ? -INFINITY : s[j][g] * scale_log2;
      }
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
          for (int u = 0; u < FQ; ++u) o[g][u] *= alpha;
          m[g] = mn;
        }
      }
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
        // a slot past the context may hold anything, NaN included, and 0 * NaN is NaN
        const bool past = tail && tb + j * TPL + r >= s1;
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          const float w = fast_exp2(s[j][g] - m[g]);
          l[g] += w;
#pragma unroll
          for (int u = 0; u < FQ; ++u) {
            const f32x4 v = past ? f32x4{0.f, 0.f, 0.f, 0.f} : vc[j][u];
            o[g][u].x = fmaf(w, v.x, o[g][u].x);
            o[g][u].y = fmaf(w, v.y, o[g][u].y);
            o[g][u].z = fmaf(w, v.z, o[g][u].z);
            o[g][u].w = fmaf(w, v.w, o[g][u].w);
          }
        }
      }
    };

    uint32_t offA[NLD], offB[NLD];
    Row kA[NLD], kB[NLD], vc[NLD];
    int ci = 0;
    offsets(0, offA);
#pragma unroll
    for (int j = 0; j < NLD; ++j) load(kbase, offA[j], kA[j]);
    while (ci < nch) {
#pragma unroll
      for (int j = 0; j < NLD; ++j) load(vbase, offA[j], vc[j]);
      if (ci + 1 < nch) {
        offsets(ci + 1, offB);
#pragma unroll
        for (int j = 0; j < NLD; ++j) load(kbase, offB[j], kB[j]);
      }
      consume(ci, kA, vc);
      if (++ci >= nch) break;
#pragma unroll
      for (int j = 0; j < NLD; ++j) load(vbase, offB[j], vc[j]);
      if (ci + 1 < nch) {
        offsets(ci + 1, offA);
#pragma unroll
        for (int j = 0; j < NLD; ++j) load(kbase, offA[j], kA[j]);
      }
      consume(ci, kB, vc);
      ++ci;
    }
  }
  if (!active) return;
  // The TPL lane groups of the wave meet (butterfly: every group ends with the merged state).
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
      for (int u = 0; u < FQ; ++u) {
        o[g][u].x = o[g][u].x * a + __shfl_xor(o[g][u].x, st) * b;
        o[g][u].y = o[g][u].y * a + __shfl_xor(o[g][u].y, st) * b;
        o[g][u].z = o[g][u].z * a + __shfl_xor(o[g][u].z, st) * b;
        o[g][u].w = o[g][u].w * a + __shfl_xor(o[g][u].w, st) * b;
      }
    }
  }
  if (r != 0) return;
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    const int head = h0 + g;
    const float inv = (l[g] > 0.f ? 1.0f / l[g] : 0.f) * p.v_scale;
    if (SPLIT && np > 1) {
      const int64_t slot = partial_index(p, row, head, np) + wg.part;
#pragma unroll
      for (int u = 0; u < FQ; ++u) *reinterpret_cast<f32x4*>(p.part_o + slot * D + c * F + 4 * u) = o[g][u] * inv;
      if (c == 0) {
        p.part_ml[slot * 2] = m[g];
        p.part_ml[slot * 2 + 1] = l[g];
      }
    } else {
#pragma unroll
      for (int u = 0; u < FQ; ++u)
        *reinterpret_cast<f32x4*>(out + ((int64_t)row * p.num_heads + head) * D + c * F + 4 * u) = o[g][u] * inv;
    }
  }
}

template <int D, int GC>
static hipError_t launch_f32_typed(const AttnParams& p, bool split, hipStream_t stream) {
  const int waves = p.num_virtual_heads < kMaxWaves ? p.num_virtual_heads : kMaxWaves;
  const int groups = (p.num_virtual_heads + waves - 1) / waves;
  const int64_t items = (split && p.work) ? p.n_work : (int64_t)p.n_rows * (split ? p.max_partitions : 1);
  const dim3 grid((unsigned)(items * groups)), block(waves * kWave);
  if (split) hipLaunchKernelGGL((paged_attention_f32_kernel<D, GC, true>), grid, block, 0, stream, p);
  else hipLaunchKernelGGL((paged_attention_f32_kernel<D, GC, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_f32_gc(const AttnParams& p, int gc, bool split, hipStream_t stream) {
  switch (gc) {
    case 1: return launch_f32_typed<D, 1>(p, split, stream);
    case 2: return launch_f32_typed<D, 2>(p, split, stream);
    case 3: return launch_f32_typed<D, 3>(p, split, stream);
    case 4: return launch_f32_typed<D, 4>(p, split, stream);
    case 5: return launch_f32_typed<D, 5>(p, split, stream);
    case 6: return launch_f32_typed<D, 6>(p, split, stream);
    case 7: return launch_f32_typed<D, 7>(p, split, stream);
    case 8: return launch_f32_typed<D, 8>(p, split, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attention_f32(const AttnParams& p, int head_dim, int gc, bool split, hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_f32_gc<64>(p, gc, split, stream);
    case 128: return launch_f32_gc<128>(p, gc, split, stream);
    case 256: return launch_f32_gc<256>(p, gc, split, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ayk
