// Paged-attention decode with the q.k contraction on the matrix cores (gfx950).
//
// Same semantics, grid and outputs as the DPP kernel in paged_attention.hip (a
// workgroup per (row, partition), one wave per key/value head); only the way a
// wave turns a chunk of 16 keys into weights differs. The library runs it from 3
// query heads per wave, and for every fp8 cache:
//
//  * Keys are loaded like the values -- 256 contiguous bytes per token, the
//    pattern HBM streams best -- and staged through a per-wave LDS tile, from
//    which each lane reads its MFMA operand: 16 bytes of token l%16 at k-slice
//    8*(l/16) of each 32-wide step (a swizzle keeps those reads conflict-free).
//  * q.k for 16 tokens x (up to 16) query heads is one 16x16 tile, accumulated
//    over head_dim by v_mfma_f32_16x16x32_{bf16,f16}: exact products, fp32
//    sums; q needs only head_dim/32 registers per lane whatever the group size.
//    Lane l gets the scores of tokens 4*(l/16)+i, i < 4, for head l%16.
//  * The softmax runs on those 4 scores per lane (max across the 4 lane
//    groups with two shuffles).
//  * P.V is O^T += V^T P^T on v_mfma_f32_16x16x16: the lane's 4 weights are
//    exactly its B operand (tokens 4*(l/16)+i of head l%16), and V^T comes from
//    a token-major LDS tile through ds_read_b64_tr_b16. A bf16 P is split into
//    a truncated high part and the remainder (two MFMAs, fp32-level accuracy;
//    one bf16 P would cost ~2e-3 relative); an fp16 P rounded to nearest is
//    within 2^-12 and takes one.
//  * fp8 caches (KV8) are decoded at their use; a chunk then holds two 16-token
//    tiles (one at head_dim 256), so a wave keeps as many bytes in flight as
//    with 16-bit caches.
//
// This removes the per-token dot2 and butterfly work that grows with the group
// in the DPP kernel, and reads keys as whole 256-byte token rows.
#include "attention_common.h"


namespace ayk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <bool BF16>
__device__ __forceinline__ f32x4 mfma_qk(u32x4 k, u32x4 q, f32x4 acc) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, k),
                                                   __builtin_bit_cast(bf16x8, q), acc, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, k),
                                                  __builtin_bit_cast(f16x8, q), acc, 0, 0, 0);
  }
}


// Order the LDS traffic of one wave: lanes read what other lanes of the same
// wave wrote just before (the wave's LDS operations execute in program order).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// WIN: a window launch (verify windows, short chunks). A work item is a tile of the
// multi-row tile list, p.work[4 * item] = (first row, rows, request, partition), of at most
// 16 / group rows of one request; p.wave_split waves serve one key/value head (taking
// every n-th chunk, merged in LDS as in v1) and their 16 MFMA columns are the tile's
// (row, query head) pairs, column mt = row mt / group, head mt % group, each masked at its
// own row's position. The context is read once for all the tile's rows. Partials (split
// launches) are merged per row by row_reduce_kernel.
template <int D, int GC, bool BF16, bool SPLIT, bool KV8, bool WIN = false>
__global__ __launch_bounds__(kMaxWaves * kWave) void paged_attention_mfma_kernel(const AttnParams p) {
  constexpr int MT = decode_tile_positions();  // tokens per MFMA tile
  // Tiles per chunk (decode_tiles_per_chunk: about as many bytes in flight per wave as a
  // 16-bit tile of head_dim 128). Measured: C2 (fp16, head_dim 64) 26.2 -> 25.2 us with two.
  constexpr int SUB = decode_tiles_per_chunk(D, KV8);
  constexpr int CH = MT * SUB;      // tokens per chunk
  constexpr int KS = D / 32;        // MFMA k-steps over head_dim
  constexpr int CPT = pieces_per_position(D);  // 8-element pieces per token (= value lanes per token)
  constexpr int TPL = positions_per_load(D);   // tokens per load instruction
  constexpr int NL1 = MT / TPL;     // load instructions per tile, for K and for V
  constexpr int NL = CH / TPL;      // load instructions per chunk
  constexpr int DT = D / 16;        // 16-element slices of head_dim for P.V
  // A tile's values in LDS, token-major, rows VP elements apart: the transposing
  // reads of one instruction (16 rows, 32 bytes each) then cover the banks evenly.
  constexpr int VP = D + 16;

  __shared__ uint32_t s_tbl[kTableCap];
  __shared__ u32x4 s_k[kMaxWaves][MT * CPT];       // a tile's keys, swizzled (see key_slot)
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kMaxWaves][MT * VP];  // a tile's values
  static_assert(SUB >= 1 && CH % TPL == 0 && NL == SUB * NL1, "chunk shape");
  __shared__ int s_last;
  // v1 with a row's context split among waves: each slice's running max and weight sum
  __shared__ float s_slice_m[kMaxWaves][16], s_slice_l[kMaxWaves][16];

  const int tid = threadIdx.x;
  const int threads = blockDim.x;
  const int waves = threads / kWave;
  // `ws` waves share one virtual head, each streaming every ws-th chunk of its context (v1)
  // or partition (v2), and their states are merged in LDS at the end: v1 fills the GPU when
  // rows x heads alone leave compute units idle, v2 covers a partition ws times as long
  // with the same per-wave work, so a row has fewer partials to store and merge.
  const int ws = p.wave_split;
  const int heads_per_wg = waves / ws;
  const int groups = (p.num_virtual_heads + heads_per_wg - 1) / heads_per_wg;
  WgCoord wg;
  int win_first = 0, win_rows = 0;  // WIN: the tile's rows
  if constexpr (WIN) {
    const int item = blockIdx.x / groups;
    win_first = p.work[4 * item];
    win_rows = p.work[4 * item + 1];
    const int size = *(p.staged ? p.staged : p.work);  // a valid stand-in address without staging
    wg = WgCoord{p.work[4 * item + 2], (int)(blockIdx.x % groups), p.work[4 * item + 3],
                 SPLIT ? (p.staged ? size : p.partition_size) : 0};
  } else {
    wg = wg_coord(p, groups, SPLIT);
    if (wg.row < 0) return;  // past the staged work items (uniform per workgroup)
  }
  const int row = wg.row;  // WIN: the request
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int vh = wg.group * heads_per_wg + wave / ws;
  const int slice = wave % ws;
  const bool active = vh < p.num_virtual_heads;
  const int kvh = vh / p.head_chunks;
  const int h0 = kvh * p.group + (vh % p.head_chunks) * GC;
  const int mt = lane % 16;  // MFMA: token of the key operand; head of q and of the scores
  const int mq = lane / 16;  // MFMA: k-slice of the operands; token group of the scores
  const int r = lane / CPT;  // loads: token within a load instruction
  const int c = lane % CPT;  // loads: 16-byte piece of head_dim

  // A token's 16-byte pieces sit in LDS at piece ^ (token % CPT): the 16 lanes that
  // read one k-slice of 16 different tokens hit 16 different bank groups.
  auto key_slot = [](int token, int piece) { return token * CPT + (piece ^ (token & (CPT - 1))); };

  int req, len;
  int win_lim = 0;        // WIN: the last position column mt's row sees
  bool win_col = false;   // WIN: column mt is a (row, head) pair of the tile
  int win_row = 0, win_head = 0;
  if constexpr (WIN) {
    req = row;
    len = max(0, min(p.kv_lengths[req], p.max_len));
    const int rr = mt / p.group;
    win_col = active && rr < win_rows;
    win_row = win_first + min(rr, win_rows - 1);
    win_head = kvh * p.group + mt % p.group;
    win_lim = len > 0 ? min(p.positions[win_row], len - 1) : 0;
    // the tile's last row sees the most; nothing past it is read (a negative position
    // leaves nothing to read: the tile's rows get zeros, as row_context gives them)
    if (len > 0) len = max(0, min(len, p.positions[win_first + win_rows - 1] + 1));
  }
  const int psize = SPLIT ? wg.psize : 0;
  // positions per staged table segment: at most kTableCap blocks, whatever s0's offset
  const int seg_len = segment_positions(p, CH);
  // Decode rows: the request, then its first table segment and its length together (the
  // segment is known from the partition alone).
  TableAhead<2> ahead;
  if constexpr (!WIN) {
    req = row_request(p, row);
    table_ahead(p, p.block_table + (int64_t)req * p.table_stride, SPLIT ? wg.part * psize : 0,
                SPLIT ? min(psize, seg_len) : seg_len, tid, threads, ahead);
    len = row_length(p, row, req);
  }
  int t_begin = 0, t_end = len;
  const int np = SPLIT ? (len > 0 ? (len - 1) / psize + 1 : 0) : 1;  // partitions with tokens
  if constexpr (WIN) {
    if (len == 0 || (SPLIT && wg.part * psize >= len)) {
      // a padding request's rows are zero (partition 0 writes them); an empty partition: nothing
      if (len == 0 && (!SPLIT || wg.part == 0) && win_col) {
        f32x4 zero[DT];
#pragma unroll
        for (int t = 0; t < DT; ++t) zero[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        store_head_t<D, BF16, false>(p, win_row, 0, 1, win_head, mq, zero, kNoScore, 0.f);
      }
      return;
    }
    if constexpr (SPLIT) {
      t_begin = wg.part * psize;
      t_end = min(len, t_begin + psize);
    }
  } else if constexpr (SPLIT) {
    t_begin = wg.part * psize;
    t_end = min(len, t_begin + psize);
    if (t_begin >= t_end) {  // only partitions that hold tokens are merged
      if (len == 0 && wg.part == 0 && active && slice == 0) store_zero_rows<D, GC, kWave>(p, row, h0, lane);
      return;
    }
  } else if (len == 0) {
    if (active && slice == 0) store_zero_rows<D, GC, kWave>(p, row, h0, lane);
    return;
  }

  // q as the MFMA B operand: head mt (zero columns past the group), k-slice mq of step s.
  u32x4 qb[KS];
  const bool q_col = WIN ? win_col : (active && mt < GC);
  const int64_t q_at = WIN ? (int64_t)win_row * p.num_heads + win_head : (int64_t)row * p.num_heads + h0 + mt;
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qb[s] = q_col ? *reinterpret_cast<const u32x4*>(p.q + q_at * D + s * 32 + mq * 8) : u32x4{0u, 0u, 0u, 0u};

  float m_h = kNoScore;  // running max of head mt (same in its 4 lanes)
  float l_h = 0.f;       // this lane's share of head mt's weight sum
  // O^T: o[t] holds elements 16t + 4*mq + i (i < 4) of head mt's unnormalised output.
  f32x4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* tbl = p.block_table + (int64_t)req * p.table_stride;
  const uint32_t token_stride = (uint32_t)p.token_stride;
  const float scale_log2 = p.scale_log2;
  const uint16_t* kbase = kv_at<KV8>(p.k_cache, (int64_t)kvh * p.head_stride + c * 8);
  const uint16_t* vbase = kv_at<KV8>(p.v_cache, (int64_t)kvh * p.head_stride + c * 8);

  for (int s0 = t_begin; s0 < t_end; s0 += seg_len) {
    const int s1 = min(t_end, s0 + seg_len);
    const int b0 = (!WIN && s0 == t_begin) ? commit_table(p, tbl, s_tbl, ahead, s1, tid, threads)
                                           : stage_table(p, tbl, s_tbl, s0, s1, tid, threads);
    const int nch = (s1 - s0 + CH - 1) / CH;
    if (!active || slice >= nch) continue;
    // this wave's chunks: slice, slice + ws, ..., up to `last`
    const int last = last_chunk_of_slice(nch, slice, ws);

    auto offsets = [&](int ci, uint32_t(&dst)[NL]) {
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        dst[j] = kv_offset(p, s_tbl, b0, chunk_position(s0, s1, ci, CH, j, TPL, r), token_stride);
      }
    };

    typedef typename KvRaw<KV8>::T Raw;
    // P.V's operand type: fp16 over fp8 caches (every e4m3 value is an fp16 value, so the
    // values decode straight to fp16 and an fp16 P rounded to nearest takes one MFMA), else the
    // model's (a bf16 P split in two)
    // (fp8 C3 89.0-89.5 -> 87.5 us, C4 partition kernel 56.5 -> 55.1, C5 226 -> 223.4)
    constexpr bool PB = KV8 ? false : BF16;
    // Fold chunk ci (keys kc, values vc) into the running state. The chunk's SUB tiles
    // share one softmax step: their keys pass through the wave's LDS tile one after the
    // other (each tile's q.k MFMAs read it before the next tile's stores, a wave's LDS
    // accesses running in program order), the SUB independent score tiles then take one
    // max, one rescale decision and one pass of exponentials, and the values follow tile
    // by tile for P.V.
    auto consume = [&](int ci, const Raw(&kc)[NL], const Raw(&vc)[NL]) {
      const int tc = s0 + ci * CH;
      const bool tail = tc + CH > s1;
      f32x4 acc[SUB];
#pragma unroll
      for (int sub = 0; sub < SUB; ++sub) {
#pragma unroll
        for (int j = 0; j < NL1; ++j) s_k[wave][key_slot(j * TPL + r, c)] = kv_pairs<KV8, BF16>(kc[sub * NL1 + j]);
        wave_lds_sync();
        acc[sub] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) acc[sub] = mfma_qk<BF16>(s_k[wave][key_slot(mt, s * 4 + mq)], qb[s], acc[sub]);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < SUB; ++sub)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = tc + sub * MT + 4 * mq + i;
          float v = acc[sub][i] * scale_log2;
          if (WIN ? (!win_col || t > win_lim) : mt >= GC) v = -INFINITY;
          if (tail && t >= s1) v = -INFINITY;
          acc[sub][i] = v;
          mx = fmaxf(mx, v);
        }
      // m_h is the same in the 4 lanes of a column, so some lane's own maximum passes it by
      // more than the slack iff some column's does: the cross-lane maximum only on a rescale
      if (__builtin_amdgcn_ballot_w64(mx > m_h + kRescaleSlack)) {
        const float mn = fmaxf(m_h, column_max(mx));
        const float alpha = fast_exp2(m_h - mn);  // head mt's, and o[] holds head mt
        l_h *= alpha;
        m_h = mn;
#pragma unroll
        for (int t = 0; t < DT; ++t) o[t] *= alpha;
      }
#pragma unroll
      for (int sub = 0; sub < SUB; ++sub) {
        float w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          w[i] = fast_exp2(acc[sub][i] - m_h);
          l_h += w[i];
        }
        // O^T += V^T P^T: P^T is the lane's own weights (tokens 4*mq + i of head mt, the
        // B operand layout); V^T comes transposed from the token-major tile (lane mt of
        // group mq reads 4 elements of token 4*mq + mt / 4). Positions past the context
        // hold real (clamped) values with weight 0.
        u32x2 phi, plo;
        split_weights4<PB>(w, phi, plo);
        // The tile's values to LDS (token-major, read back transposed) only now: their
        // loads were issued with this chunk's, and the wait for them overlaps q.k and
        // the softmax (C2 24.7 -> 24.0 us, fp8 C3 87.7 -> 86.2 us).
#pragma unroll
        for (int j = 0; j < NL1; ++j)
          *reinterpret_cast<u32x4*>(&s_v[wave][(j * TPL + r) * VP + c * 8]) = kv_pairs<KV8, PB>(vc[sub * NL1 + j]);
        wave_lds_sync();
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const u32x2 va = lds_read_transposed(&s_v[wave][(4 * mq + (mt >> 2)) * VP + t * 16 + 4 * (mt & 3)]);
          o[t] = mfma_pv<PB>(va, phi, o[t]);
          if constexpr (split_p(PB)) o[t] = mfma_pv<PB>(va, plo, o[t]);
        }
      }
    };

    // Keys of the next chunk are in flight while the current one is folded in. The
    // prefetch is unconditional -- at the last chunk it re-reads that chunk, which
    // has just arrived -- so the compiler's waits for the values before each use
    // leave the next chunk's keys outstanding (a conditional load would make them
    // wait for everything).
    uint32_t offA[NL], offB[NL];
    Raw kA[NL], kB[NL], vc[NL];
    int ci = slice;
    offsets(ci, offA);
#pragma unroll
    for (int j = 0; j < NL; ++j) kA[j] = load_kv_raw<KV8>(kbase, offA[j]);
    while (ci <= last) {
#pragma unroll
      for (int j = 0; j < NL; ++j) vc[j] = load_kv_raw<KV8>(vbase, offA[j]);
      offsets(min(ci + ws, last), offB);
#pragma unroll
      for (int j = 0; j < NL; ++j) kB[j] = load_kv_raw<KV8>(kbase, offB[j]);
      consume(ci, kA, vc);
      ci += ws;
      if (ci > last) break;
#pragma unroll
      for (int j = 0; j < NL; ++j) vc[j] = load_kv_raw<KV8>(vbase, offB[j]);
      offsets(min(ci + ws, last), offA);
#pragma unroll
      for (int j = 0; j < NL; ++j) kA[j] = load_kv_raw<KV8>(kbase, offA[j]);
      consume(ci, kB, vc);
      ci += ws;
    }
  }
  // Head mt's weight sum over the wave's 4 token groups (its lanes share m_h).
  l_h += __shfl_xor(l_h, 16);
  l_h += __shfl_xor(l_h, 32);
  if (ws > 1) {
    // Slices 1.. of a head hand (m, l, o) to slice 0 through their own LDS tiles (the
    // keys' tile takes o[0, DT/2), the values' tile the rest: 4 * D 16-byte entries fit
    // in 2 * D + (D + 16) / 4), which folds them in slice order: the result does not
    // depend on the waves' timing.
    constexpr int HALF = DT / 2;
    u32x4* vt = reinterpret_cast<u32x4*>(&s_v[wave][0]);
    if (active && slice > 0) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const u32x4 w = __builtin_bit_cast(u32x4, o[t]);
        if (t < HALF) s_k[wave][t * kWave + lane] = w;
        else vt[(t - HALF) * kWave + lane] = w;
      }
      if (lane < 16) {
        s_slice_m[wave][lane] = m_h;
        s_slice_l[wave][lane] = l_h;
      }
    }
    __syncthreads();
    if (active && slice == 0) {
      for (int j = 1; j < ws; ++j) {
        const int src = wave + j;
        const float mj = s_slice_m[src][mt], lj = s_slice_l[src][mt];
        const float mn = fmaxf(m_h, mj);
        const float a = fast_exp2(m_h - mn), b = fast_exp2(mj - mn);
        l_h = l_h * a + lj * b;
        m_h = mn;
        const u32x4* vs = reinterpret_cast<const u32x4*>(&s_v[src][0]);
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const f32x4 oj = __builtin_bit_cast(f32x4, t < HALF ? s_k[src][t * kWave + lane]
                                                              : vs[(t - HALF) * kWave + lane]);
          o[t] = o[t] * a + oj * b;
        }
      }
    }
  }
  if (active && slice == 0) {
    if constexpr (WIN) {
      // the row sees positions [0, win_lim]: partitions past it hold nothing of it
      const int np_row = SPLIT ? win_lim / psize + 1 : 1;
      if (win_col && wg.part < np_row)
        store_head_t<D, BF16, SPLIT>(p, win_row, wg.part, np_row, win_head, mq, o, m_h, l_h);
    } else if (mt < GC) {
      store_head_t<D, BF16, SPLIT>(p, row, wg.part, np, h0 + mt, mq, o, m_h, l_h);
    }
  }
  if constexpr (SPLIT && !WIN) {
    if (np > 1 && p.arrivals) {
      const int vh_lo = wg.group * heads_per_wg;
      const int vh_hi = min(p.num_virtual_heads, vh_lo + heads_per_wg);
      arrive_and_merge<D, GC, BF16>(p, row, wg.group, groups, np, vh_lo * GC, vh_hi * GC, tid, threads, &s_last);
    }
  }
}

template <int D, int GC, bool BF16, bool KV8>
static hipError_t launch_mfma_typed(const AttnParams& p, bool split, hipStream_t stream) {
  // p.wave_split waves per virtual head, up to kMaxWaves per workgroup
  const int ws = p.wave_split;
  const int heads = p.num_virtual_heads < kMaxWaves / ws ? p.num_virtual_heads : kMaxWaves / ws;
  const int per_wg = heads * ws;
  const int groups = (p.num_virtual_heads + heads - 1) / heads;
  const int64_t items = (split && p.work) ? p.n_work : (int64_t)p.n_rows * (split ? p.max_partitions : 1);
  const dim3 grid((unsigned)(items * groups)), block(per_wg * kWave);
  if (split)
    hipLaunchKernelGGL((paged_attention_mfma_kernel<D, GC, BF16, true, KV8>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((paged_attention_mfma_kernel<D, GC, BF16, false, KV8>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <int D, bool BF16, bool KV8>
static hipError_t launch_mfma_gc(const AttnParams& p, int gc, bool split, hipStream_t stream) {
  switch (gc) {
    case 1: return launch_mfma_typed<D, 1, BF16, KV8>(p, split, stream);
    case 2: return launch_mfma_typed<D, 2, BF16, KV8>(p, split, stream);
    case 3: return launch_mfma_typed<D, 3, BF16, KV8>(p, split, stream);
    case 4: return launch_mfma_typed<D, 4, BF16, KV8>(p, split, stream);
    case 5: return launch_mfma_typed<D, 5, BF16, KV8>(p, split, stream);
    case 6: return launch_mfma_typed<D, 6, BF16, KV8>(p, split, stream);
    case 7: return launch_mfma_typed<D, 7, BF16, KV8>(p, split, stream);
    case 8: return launch_mfma_typed<D, 8, BF16, KV8>(p, split, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int D>
static hipError_t launch_mfma_d(const AttnParams& p, int gc, bool bf16, bool split, bool kv8, hipStream_t stream) {
  if (kv8) return bf16 ? launch_mfma_gc<D, true, true>(p, gc, split, stream)
                       : launch_mfma_gc<D, false, true>(p, gc, split, stream);
  return bf16 ? launch_mfma_gc<D, true, false>(p, gc, split, stream)
              : launch_mfma_gc<D, false, false>(p, gc, split, stream);
}

template <int D, bool BF16, bool KV8>
static hipError_t launch_window_typed(const AttnParams& p, bool split, hipStream_t stream) {
  // p.wave_split waves per key/value head, up to kMaxWaves per workgroup; 16 MFMA columns per wave
  const int ws = p.wave_split;
  const int heads = p.num_virtual_heads < kMaxWaves / ws ? p.num_virtual_heads : kMaxWaves / ws;
  const int per_wg = heads * ws;
  const int groups = (p.num_virtual_heads + heads - 1) / heads;
  const dim3 grid((unsigned)((int64_t)p.n_work * groups)), block(per_wg * kWave);
  if (split)
    hipLaunchKernelGGL((paged_attention_mfma_kernel<D, 16, BF16, true, KV8, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((paged_attention_mfma_kernel<D, 16, BF16, false, KV8, true>), grid, block, 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_window_mfma(const AttnParams& p, int head_dim, bool bf16, bool split, bool kv8, hipStream_t stream) {
  switch (head_dim) {
    case 64:
      if (kv8) return bf16 ? launch_window_typed<64, true, true>(p, split, stream)
                           : launch_window_typed<64, false, true>(p, split, stream);
      return bf16 ? launch_window_typed<64, true, false>(p, split, stream)
                  : launch_window_typed<64, false, false>(p, split, stream);
    case 128:
      if (kv8) return bf16 ? launch_window_typed<128, true, true>(p, split, stream)
                           : launch_window_typed<128, false, true>(p, split, stream);
      return bf16 ? launch_window_typed<128, true, false>(p, split, stream)
                  : launch_window_typed<128, false, false>(p, split, stream);
    case 256:
      if (kv8) return bf16 ? launch_window_typed<256, true, true>(p, split, stream)
                           : launch_window_typed<256, false, true>(p, split, stream);
      return bf16 ? launch_window_typed<256, true, false>(p, split, stream)
                  : launch_window_typed<256, false, false>(p, split, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attention_mfma(const AttnParams& p, int head_dim, int gc, bool bf16, bool split, bool kv8,
                                 int waves, hipStream_t stream) {
  (void)waves;
  switch (head_dim) {
    case 64: return launch_mfma_d<64>(p, gc, bf16, split, kv8, stream);
    case 128: return launch_mfma_d<128>(p, gc, bf16, split, kv8, stream);
    case 256: return launch_mfma_d<256>(p, gc, bf16, split, kv8, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ayk
