// Multi-row paged attention (prefill chunks, verify windows) on the matrix cores (gfx950).
//
// Semantics: the reference's multi-row rule (python/ayaka/ops/backends/torch/
// attention.py:209-234): the rows of a request are its last rows, row j at
// position p_j attends to positions [0, p_j] of the request's paged context,
// scores scale * q.k, softmax and P.V in fp32, the output rounded once; rows of a
// padding request (kv_lengths 0) are zero.
//
// A workgroup of 4 waves serves one tile: up to TILE_PAIRS (row, query head)
// pairs of one request and one key/value head -- the TILE_PAIRS / G consecutive
// rows of the request whose G query heads read that key/value head. Each wave
// owns PT groups of 16 pairs. The context streams through LDS in chunks of 64
// positions (32 at head_dim 256 with 1 or 2 waves per pair group), loaded once
// per tile, cooperatively, one chunk ahead in registers.
// A launch with partitions (p.part_o set) gives each tile one workgroup per
// partition of p.partition_size positions (a multiple of 64); a row's partitions
// store v2 partials (the output itself when the row has one partition) for
// partition_reduce_kernel to merge.
//
//  * S^T = K Q^T, per 16-position tile and 16-pair group: v_mfma_f32_16x16x32
//    over head_dim, keys from a swizzled LDS tile (A operand), q from registers
//    (B operand). Lane l holds the scores of positions 4*(l/16)+i of pair l%16,
//    so every per-pair quantity (running max, weight sum, rescale) lives in the
//    lane's own column.
//  * O^T += V^T P^T, per 16-element slice of head_dim and 32 positions:
//    v_mfma_f32_16x16x32 with P^T taken straight from the lane's scores (its
//    8 k-slots are positions 4*(l/16)+i of two adjacent 16-position tiles) and
//    V^T read in that same position order from a token-major LDS tile through
//    ds_read_b64_tr_b16 (two 4-position reads per operand). A bf16 P is
//    split by truncation into a 16-bit high part and the 16-bit remainder, two
//    MFMAs, which keeps the product at fp32-level accuracy (one bf16 P would cost
//    ~2e-3 relative); an fp16 P rounded to nearest is within 2^-12 and takes one.
//  * Keys and values are staged with 16-byte LDS stores, values token-major in
//    rows D + 16 elements apart, which keeps the transposing reads of a 16-lane
//    group spread over the banks.
#include "attention_common.h"


namespace ayk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kPrefillWaves = 4;

// (row, head) pairs one workgroup serves: 2 groups of 16 per wave, 1 at head_dim 256
// (the accumulators of 2 groups would not fit the register file there).
__host__ __device__ constexpr int prefill_tile_pairs(int head_dim) {
  return kPrefillWaves * 16 * (head_dim == 256 ? 1 : 2);
}

template <bool BF16>
__device__ __forceinline__ f32x4 mfma32(u32x4 a, u32x4 b, f32x4 acc) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   acc, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                  acc, 0, 0, 0);
}

// Split 8 fp32 weights w (finite, >= 0) as split_weights4 (bf16: high parts and
// remainders by truncation, one v_perm_b32 packing two; fp16: rounded to nearest).
template <bool BF16>
__device__ __forceinline__ void split_weights(const float (&w)[8], u32x4& hi, u32x4& lo) {
  u32x2 h0, l0, h1, l1;
  split_weights4<BF16>({w[0], w[1], w[2], w[3]}, h0, l0);
  split_weights4<BF16>({w[4], w[5], w[6], w[7]}, h1, l1);
  hi = u32x4{h0.x, h0.y, h1.x, h1.y};
  lo = u32x4{l0.x, l0.y, l1.x, l1.y};
}

// Workgroups per CU the register budget is set for: two, except quarter tiles at head_dim 256,
// whose 64-position stage (133 KB of LDS) leaves room for one.
__host__ __device__ constexpr int prefill_workgroups_per_cu(int head_dim, int waves_per_group) {
  return head_dim == 256 && waves_per_group == 4 ? 1 : 2;
}

// W: waves per workgroup, kPrefillWaves, or 8 for the double tile (head_dim 128 and 256, one
// workgroup per CU): one stage of each chunk then serves 8 waves' pairs, which halves the
// staging loads, LDS writes and barrier per pair (4 x 512 rows over 4K, settled: 174.5 -> 171.5
// us; GQA 8 335 -> 322; fp16 140 -> 135; head_dim 256 208 -> 193).
//
// MODE (bf16 models over bf16 caches; 0 otherwise): P.V costs two MFMAs per step for a bf16 P
// (its split) but one for an fp16 P rounded to nearest, which needs the values in fp16. Every
// bf16 value with 2^-17 <= |v| < 65536 is an fp16 value (fp16's normal range, and the
// subnormals that still hold bf16's 8 significant bits); smaller ones round to within 2^-25.
// MODE 1 stages each chunk's values as fp16 and votes: a chunk holding a value of 65536 or more
// (or not finite), or none of 2^-10 or more (where the small values' rounding could matter),
// does not convert. A workgroup that met such a chunk stores nothing and marks its slot of
// p.arrivals, which MODE 1 otherwise clears at its start. MODE 2, launched after it on the
// same grid, runs only the marked workgroups, with the split bf16 P. fp8 caches decode
// straight to fp16 (every e4m3 value is one), so bf16 models over them always take one MFMA.
template <int D, bool BF16, bool KV8, int PS, int W = kPrefillWaves, int MODE = 0>
__global__ __launch_bounds__(W * kWave, W == 8 ? 1 : prefill_workgroups_per_cu(D, PS)) void paged_prefill_kernel(
    const AttnParams p, const int32_t* tiles) {
  static_assert(W == kPrefillWaves || (W == 8 && PS == 1 && D != 64), "the double tile: 8 waves, one per pair group");
  static_assert(MODE == 0 || (BF16 && !KV8), "the fp16 values pass: bf16 models over bf16 caches");
  constexpr bool V16_ALWAYS = KV8 && BF16;  // fp8 codes decode to fp16 values
  constexpr bool V16_FAST = MODE == 1;      // bf16 values, staged as fp16 when they all convert
  constexpr bool V16 = V16_ALWAYS || V16_FAST;
  if constexpr (MODE == 2) {
    if (p.arrivals[blockIdx.x] == 0) return;  // the fast pass finished this workgroup (uniform)
  }
  if constexpr (MODE == 1) {
    if (threadIdx.x == 0) p.arrivals[blockIdx.x] = 0;
  }
  constexpr int THREADS = W * kWave;
  constexpr int PT = D == 256 ? 1 : 2;          // 16-pair groups per wave
  constexpr int PGROUPS = W / PS;               // waves with distinct pairs
  constexpr int TILE_PAIRS = prefill_tile_pairs(D) * (W / kPrefillWaves) / PS;
  // Positions per chunk: 64, or 32 at head_dim 256 with 1 or 2 waves per pair group, where a
  // 64-position stage (133 KB of LDS) and its load registers left one wave per SIMD; 32 fit
  // two workgroups per CU without spills (quarter tiles need 16 positions per wave: 64).
  constexpr int CH = prefill_chunk_positions(D, PS);
  constexpr int PTL = CH / 16;                  // 16-position tiles per chunk
  constexpr int PTL_W = PTL / PS;               // 16-position tiles per chunk of one wave
  constexpr int KS = D / 32;                    // q.k k-steps
  constexpr int DT = D / 16;                    // 16-element slices of head_dim for P.V
  constexpr int CPT = pieces_per_position(D);   // 8-element pieces per position
  constexpr int PIECES = CH * CPT;              // pieces per chunk of K (or V)
  constexpr int PER_THREAD = PIECES / THREADS;  // 2 (D 64), 4 (D 128), 4 or 8 (D 256); half with 8 waves
  // Values in LDS token-major, rows VP elements apart: the transposing reads of the
  // P.V operand (16 rows of one 16-lane group, 8 bytes each) then cover the banks evenly.
  constexpr int VP = D + 16;
  static_assert(PER_THREAD % 2 == 0 && PIECES % THREADS == 0, "piece split");
  static_assert(PS == 1 || PS == 2 || PS == 4, "waves per pair group");

  // The staged chunks, and after the last one the running states the waves of a
  // group with ps > 0 hand to its first wave: o of each lane, m and l per pair.
  struct Stage {
    u32x4 k[2][PIECES];
    uint16_t v[2][CH * VP];
  };
  constexpr int MERGE_WAVES = PS > 1 ? (PS - 1) * PGROUPS : 1;
  union Lds {
    Stage st;
    f32x4 o[MERGE_WAVES][PT][DT][kWave];
  };
  static_assert(sizeof(f32x4[MERGE_WAVES][PT][DT][kWave]) <= sizeof(Stage), "merge fits the stage");
  __shared__ uint32_t s_tbl[kTableCap];
  __shared__ Lds lds;
  __shared__ float s_ml[MERGE_WAVES][PT][2][16];
  __shared__ int s_vbad[2][W];  // V16_FAST: per buffer, each wave's vote (a value that does not convert)
  auto& s_k = lds.st.k;
  auto& s_v = lds.st.v;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int pg = wave / PS;  // this wave's pair group
  const int ps = wave % PS;  // and its share of each chunk: tiles ps * PTL_W ...
  const int mt = lane % 16;
  const int mq = lane / 16;
  const int kv_heads = p.num_heads / p.group;
  const int kvh = blockIdx.x % kv_heads;
  const int tile = blockIdx.x / kv_heads;
  const int first_row = tiles[4 * tile];
  const int group = p.group;
  const int n_pairs = min(tiles[4 * tile + 1] * group, TILE_PAIRS);
  const int n_rows = (n_pairs + group - 1) / group;
  const int req = tiles[4 * tile + 2];
  const bool split = p.part_o != nullptr;
  const int part = split ? tiles[4 * tile + 3] : 0;

  // This lane's (row, query head) pair of each of its groups.
  bool real[PT];
  int prow[PT], phead[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    const int pair = (pg * PT + j) * 16 + mt;
    real[j] = pair < n_pairs;
    prow[j] = first_row + (real[j] ? pair / group : 0);
    phead[j] = kvh * group + (real[j] ? pair % group : 0);
  }

  int kv_len = p.kv_lengths[req];
  kv_len = max(0, min(kv_len, p.max_len));
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
  const int last_pos = min(p.positions[first_row + n_rows - 1], kv_len - 1);
  // Idle pairs (past the tile's rows) see everything: their results are not stored, and
  // they must not force the masked path on chunks every real pair sees whole.
  int my_pos[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) my_pos[j] = real[j] ? min(p.positions[prow[j]], kv_len - 1) : last_pos;
  // The earliest position any pair of this wave stops at: chunks ending at or
  // before it need no causal mask.
  int wave_min_pos = my_pos[0];
#pragma unroll
  for (int j = 1; j < PT; ++j) wave_min_pos = min(wave_min_pos, my_pos[j]);
#pragma unroll
  for (int st = 1; st < kWave; st <<= 1) wave_min_pos = min(wave_min_pos, __shfl_xor(wave_min_pos, st));

  // q as the B operand of S^T = K Q^T: pair mt of group j, k-slice mq of step s.
  u32x4 qb[PT][KS];
#pragma unroll
  for (int j = 0; j < PT; ++j)
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qb[j][s] = real[j] ? *reinterpret_cast<const u32x4*>(p.q + ((int64_t)prow[j] * p.num_heads + phead[j]) * D +
                                                           s * 32 + mq * 8)
                         : u32x4{0u, 0u, 0u, 0u};

  float m[PT], l[PT];
  // LSUM_MFMA: each pair's weight sum accumulates on the matrix cores, as one more 16-row slice
  // of O^T whose A operand is a row of ones (row 0; the other rows zero): the sum of exactly
  // the weights the P.V products use, for one MFMA per k-step and group instead of a VALU add
  // per weight. Measured on 4 x 512 rows over 4K (settled, us): head_dim 64 fp16 91.9 -> 87.5,
  // head_dim 256 187 -> 183; at head_dim 128 in the double tile over 16-bit caches bf16
  // 138.0 -> 137.0, GQA 8 260.4 -> 257.4, fp16 130.6 -> 130.2, but over fp8 caches 120.1 ->
  // 122.9 and on half tiles (the 2048-row prompt) 68.1 -> 68.9, and the full tile's fp16
  // values pass would spill, so it stays off for those.
  constexpr bool LSUM_MFMA = PTL_W >= 2 && (D != 128 || (W == 8 && !KV8));
  f32x4 lo1[PT];
  f32x4 o[PT][DT];
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    m[j] = kNoScore;
    l[j] = 0.f;
    lo1[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < DT; ++t) o[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int32_t* tbl = p.block_table + (int64_t)req * p.table_stride;
  // positions per staged table segment: at most kTableCap blocks, whatever s0's offset
  const int seg_len = segment_positions(p, CH);
  const uint32_t token_stride = (uint32_t)p.token_stride;
  const float scale_log2 = p.scale_log2;
  const uint16_t* kbase = kv_at<KV8>(p.k_cache, (int64_t)kvh * p.head_stride);
  const uint16_t* vbase = kv_at<KV8>(p.v_cache, (int64_t)kvh * p.head_stride);
  auto key_slot = [](int token, int piece) { return token * CPT + (piece ^ (token & (CPT - 1))); };
  // Piece u of this thread: 8-element slice piece_c of the chunk's position
  // first_pos + u; consecutive threads read consecutive slices of one position, and a
  // thread's PER_THREAD positions are consecutive (one block when the block size is a
  // multiple of PER_THREAD, so one table lookup serves them all).
  const int piece_c = tid % CPT;
  const int first_pos = PER_THREAD * (tid / CPT);
  static_assert(PER_THREAD * (THREADS / CPT) == CH, "a chunk's positions, PER_THREAD per thread");

  // This workgroup's positions: the tile's whole context, or one partition of it.
  const int t_begin = split ? part * p.partition_size : 0;
  const int t_end = split ? min(last_pos + 1, t_begin + p.partition_size) : last_pos + 1;
  // V16_FAST: a chunk whose values did not all convert (uniform); its results are then not
  // stored, and the fallback pass computes the workgroup (the rest of the chunks still run:
  // leaving the loop early costs the common case registers)
  bool stop = false;
  for (int s0 = t_begin; s0 < t_end; s0 += seg_len) {
    const int s1 = min(t_end, s0 + seg_len);
    const int b0 = stage_table(p, tbl, s_tbl, s0, s1, tid, THREADS);
    const int nch = (s1 - s0 + CH - 1) / CH;

    typedef typename KvRaw<KV8>::T Raw;
    Raw kr[PER_THREAD], vr[PER_THREAD];
    // Chunk ci into registers kr and vr (K and V pieces of a position share its offset).
    // Positions past the segment's last one are read as that one (weight 0, finite
    // values). Block sizes that are a multiple of PER_THREAD (uniform across the launch)
    // take one table lookup per chunk for the thread's positions, the others one per
    // position.
    auto load_chunk = [&](int ci) {
      uint32_t off[PER_THREAD];
      prefill_offsets<PER_THREAD>(p, s_tbl, b0, s0 + ci * CH + first_pos, s1, piece_c, token_stride, off);
#pragma unroll
      for (int u = 0; u < PER_THREAD; ++u) {
        kr[u] = load_kv_raw<KV8, false>(kbase, off[u]);
        vr[u] = load_kv_raw<KV8, false>(vbase, off[u]);
      }
    };
    auto stage_keys = [&](int buf) {
#pragma unroll
      for (int u = 0; u < PER_THREAD; ++u) s_k[buf][key_slot(first_pos + u, piece_c)] = kv_pairs<KV8, BF16>(kr[u]);
    };
    auto stage_values = [&](int buf) {
      typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
      u16x2 hi_bits = {0, 0};  // V16_FAST: the largest |bits| of the thread's values
#pragma unroll
      for (int u = 0; u < PER_THREAD; ++u) {
        u32x4 w = kv_pairs<KV8, V16_ALWAYS ? false : BF16>(vr[u]);
        if constexpr (V16_FAST) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const u16x2 a = __builtin_bit_cast(u16x2, w[e] & 0x7fff7fffu);
            hi_bits = __builtin_elementwise_max(hi_bits, a);
            // bf16 -> fp32 -> fp16, to nearest: exact from 2^-17 up, within 2^-25 below
            w[e] = __builtin_bit_cast(uint32_t, f16x2{(_Float16)__uint_as_float(w[e] << 16),
                                                      (_Float16)__uint_as_float(w[e] & 0xffff0000u)});
          }
        }
        *reinterpret_cast<u32x4*>(&s_v[buf][(first_pos + u) * VP + piece_c * 8]) = w;
      }
      if constexpr (V16_FAST) {
        // 2: a value fp16 cannot hold (|v| >= 65536, or not finite); 1: none of the wave's
        // values reaches 2^-10 (a chunk all of whose waves say so does not convert either)
        const unsigned top = max(hi_bits.x, hi_bits.y);
        const uint64_t no = __builtin_amdgcn_ballot_w64(top > 0x477f);
        const uint64_t sized = __builtin_amdgcn_ballot_w64(top >= 0x3a80);
        if (lane == 0) s_vbad[buf][wave] = no != 0 ? 2 : sized == 0 ? 1 : 0;
      }
    };

    typedef f32x4 Scores[PTL_W][PT];
    // This wave's raw scores of the chunk whose keys sit in LDS buffer kb.
    auto scores = [&](int kb, Scores& acc) {
#pragma unroll
      for (int w = 0; w < PTL_W; ++w)
#pragma unroll
        for (int j = 0; j < PT; ++j) acc[w][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int w = 0; w < PTL_W; ++w) {
          const int pt = ps * PTL_W + w;
          const u32x4 ka = s_k[kb][key_slot(pt * 16 + mt, s * 4 + mq)];
#pragma unroll
          for (int j = 0; j < PT; ++j) acc[w][j] = mfma32<BF16>(ka, qb[j][s], acc[w][j]);
        }
    };
    // Fold chunk ci's scores acc (its values in LDS buffer vb) into every pair's running
    // state; mid() runs between the rescale and the weights.
    // P.V's operand type: fp16 when the values in LDS are fp16 values, else the model's
    constexpr bool PB = V16 ? false : BF16;
    auto fold = [&](int ci, int vb, Scores& acc, auto&& mid) {
      const int buf = vb;
      const int tb = s0 + ci * CH;
      // uniform: no position masked (and, for folding the scale into the exponent,
      // a scale >= 0, under which the largest raw score gives the largest scaled one)
      const bool whole = tb + CH <= s1 && tb + CH - 1 <= wave_min_pos && scale_log2 >= 0.f;
      // the scale applied to a score in the exponent below (1 once the scores are scaled)
      const float sc = whole ? scale_log2 : 1.f;
#pragma unroll
      for (int j = 0; j < PT; ++j) {
        float mx = -INFINITY;
        if (whole) {
#pragma unroll
          for (int w = 0; w < PTL_W; ++w)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, acc[w][j][i]);
          mx *= scale_log2;
        } else {
          // position tb + pt*16 + 4*mq + i is visible iff pt*16 + i <= lim
          const int lim = min(my_pos[j], s1 - 1) - tb - 4 * mq;
#pragma unroll
          for (int w = 0; w < PTL_W; ++w)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int pt = ps * PTL_W + w;
              acc[w][j][i] = pt * 16 + i <= lim ? acc[w][j][i] * scale_log2 : -INFINITY;
              mx = fmaxf(mx, acc[w][j][i]);
            }
        }
        // m[j] is the same in the 4 lanes of a column, so some lane's own maximum passes it
        // by more than the slack iff some column's does: the cross-lane maximum only on a
        // rescale
        if (__builtin_amdgcn_ballot_w64(mx > m[j] + kRescaleSlack)) {
          const float mn = fmaxf(m[j], column_max(mx));
          const float alpha = fast_exp2(m[j] - mn);
          l[j] *= alpha;
          if constexpr (LSUM_MFMA) lo1[j] *= alpha;
#pragma unroll
          for (int t = 0; t < DT; ++t) o[j][t] *= alpha;
          m[j] = mn;
        }
      }
      mid();
      // Weights after every group's max and rescale: from here to the end of the chunk
      // the code has no branch, so the scheduler can overlap one group's exponentials
      // with the other's P.V MFMAs.
#pragma unroll
      for (int j = 0; j < PT; ++j)
#pragma unroll
        for (int w = 0; w < PTL_W; ++w)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = fast_exp2(__builtin_fmaf(acc[w][j][i], sc, -m[j]));
            acc[w][j][i] = e;
            if constexpr (!LSUM_MFMA) l[j] += e;
          }
      if constexpr (PTL_W >= 2) {
        // O^T += V^T P^T over this wave's 32-position k-steps (16x16x32).
#pragma unroll
        for (int kw = 0; kw < PTL_W / 2; ++kw) {
          const int ks = ps * (PTL_W / 2) + kw;
          u32x4 phi[PT], plo[PT];
#pragma unroll
          for (int j = 0; j < PT; ++j) {
            const float w[8] = {acc[2 * kw][j][0],     acc[2 * kw][j][1],     acc[2 * kw][j][2],
                                acc[2 * kw][j][3],     acc[2 * kw + 1][j][0], acc[2 * kw + 1][j][1],
                                acc[2 * kw + 1][j][2], acc[2 * kw + 1][j][3]};
            split_weights<PB>(w, phi[j], plo[j]);
          }
          if constexpr (LSUM_MFMA) {
            // the ones slice: lanes of row 0 (l % 16 == 0) hold eight ones of P.V's operand type
            const uint32_t one2 = (mt == 0) ? (PB ? 0x3f803f80u : 0x3c003c00u) : 0u;
            const u32x4 ones = u32x4{one2, one2, one2, one2};
#pragma unroll
            for (int j = 0; j < PT; ++j) {
              lo1[j] = mfma32<PB>(ones, phi[j], lo1[j]);
              if constexpr (split_p(PB)) lo1[j] = mfma32<PB>(ones, plo[j], lo1[j]);
            }
          }
#pragma unroll
          for (int t = 0; t < DT; ++t) {
            // lane (mq, mt) gets element t*16 + mt of positions ks*32 + 4*mq + i (lo4)
            // and ks*32 + 16 + 4*mq + i (hi4): the order of its weights
            const uint16_t* vrow = &s_v[buf][(ks * 32 + 4 * mq + (mt >> 2)) * VP + t * 16 + 4 * (mt & 3)];
            const u32x2 lo4 = lds_read_transposed(vrow);
            const u32x2 hi4 = lds_read_transposed(vrow + 16 * VP);
            const u32x4 va = u32x4{lo4.x, lo4.y, hi4.x, hi4.y};
#pragma unroll
            for (int j = 0; j < PT; ++j) {
              o[j][t] = mfma32<PB>(va, phi[j], o[j][t]);
              if constexpr (split_p(PB)) o[j][t] = mfma32<PB>(va, plo[j], o[j][t]);
            }
          }
        }
      } else {
        // One 16-position tile per wave: O^T += V^T P^T on 16x16x16, the lane's 4
        // weights (positions 4*mq + i of the tile) as its k-slots.
        u32x2 phi[PT], plo[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) {
          const float w[4] = {acc[0][j][0], acc[0][j][1], acc[0][j][2], acc[0][j][3]};
          split_weights4<PB>(w, phi[j], plo[j]);
        }
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const u32x2 va = lds_read_transposed(&s_v[buf][(ps * 16 + 4 * mq + (mt >> 2)) * VP + t * 16 + 4 * (mt & 3)]);
#pragma unroll
          for (int j = 0; j < PT; ++j) {
            o[j][t] = mfma_pv<PB>(va, phi[j], o[j][t]);
            if constexpr (split_p(PB)) o[j][t] = mfma_pv<PB>(va, plo[j], o[j][t]);
          }
        }
      }
    };

    load_chunk(0);
    stage_keys(0);
    stage_values(0);
    lds_barrier();
    // Two chunks per iteration, so that each body's LDS buffer is a constant (immediate
    // address offsets instead of per-access arithmetic).
    // V16_FAST: whether a chunk's values all converted (every wave's vote, uniform)
    auto values_convert = [&](int buf) {
      int no = 0, small = 1;
#pragma unroll
      for (int v = 0; v < W; ++v) {
        no |= s_vbad[buf][v] & 2;
        small &= s_vbad[buf][v];
      }
      return no == 0 && small == 0;
    };
    auto chunk_step = [&](int ci, int buf) {
      if (ci + 1 < nch) load_chunk(ci + 1);
      // The two waves a SIMD holds (one per workgroup) take turns: a wave raises its
      // priority over its MFMA sections -- the q.k, and the weights with the P.V -- so
      // that its matrix instructions issue ahead of the other wave's max and rescale
      // VALU work, which fills the issue slots between them (5-6% on prefill chunks).
      Scores acc;
      __builtin_amdgcn_s_setprio(1);
      scores(buf, acc);
      __builtin_amdgcn_s_setprio(0);
      fold(ci, buf, acc, [] { __builtin_amdgcn_s_setprio(1); });
      __builtin_amdgcn_s_setprio(0);
      if (ci + 1 < nch) {
        stage_keys(buf ^ 1);
        stage_values(buf ^ 1);
      }
      lds_barrier();
    };
    for (int ci = 0; ci < nch; ci += 2) {
      if constexpr (V16_FAST) stop |= !values_convert(0);
      chunk_step(ci, 0);
      if (ci + 1 < nch) {
        if constexpr (V16_FAST) stop |= !values_convert(1);
        chunk_step(ci + 1, 1);
      }
    }
  }

  if (stop) {
    if (tid == 0) p.arrivals[blockIdx.x] = 1;
    return;
  }
  // Each pair's weight sum over the 4 position groups; lane (mq, mt) holds
  // elements 16*t + 4*mq + i of pair mt of each group.
  float lsum[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    if constexpr (LSUM_MFMA) {
      lsum[j] = __shfl(lo1[j][0], mt);  // row 0 of the ones slice: lane (0, mt)
    } else {
      lsum[j] = l[j];
      lsum[j] += __shfl_xor(lsum[j], 16);
      lsum[j] += __shfl_xor(lsum[j], 32);
    }
  }
  if constexpr (PS > 1) {
    // The waves ps > 0 of a group hand their states to wave ps = 0, which folds them
    // in: o = sum o_w 2^(m_w - M), l = sum l_w 2^(m_w - M), M = max m_w. The last
    // loop iteration ended on a barrier, so the stage area is free.
    if (ps > 0) {
      const int slot = pg * (PS - 1) + ps - 1;
#pragma unroll
      for (int j = 0; j < PT; ++j) {
#pragma unroll
        for (int t = 0; t < DT; ++t) lds.o[slot][j][t][lane] = o[j][t];
        if (mq == 0) {
          s_ml[slot][j][0][mt] = m[j];
          s_ml[slot][j][1][mt] = lsum[j];
        }
      }
    }
    lds_barrier();
    if (ps > 0) return;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      float mn = m[j];
#pragma unroll
      for (int w = 1; w < PS; ++w) mn = fmaxf(mn, s_ml[pg * (PS - 1) + w - 1][j][0][mt]);
      const float a0 = fast_exp2(m[j] - mn);
      lsum[j] *= a0;
#pragma unroll
      for (int t = 0; t < DT; ++t) o[j][t] *= a0;
#pragma unroll
      for (int w = 1; w < PS; ++w) {
        const int slot = pg * (PS - 1) + w - 1;
        const float a = fast_exp2(s_ml[slot][j][0][mt] - mn);
        lsum[j] += s_ml[slot][j][1][mt] * a;
#pragma unroll
        for (int t = 0; t < DT; ++t) o[j][t] += lds.o[slot][j][t][lane] * a;
      }
      m[j] = mn;
    }
  }
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    const float lj = lsum[j];
    if (!real[j]) continue;
    if (split) {
      // the row sees positions [0, my_pos]: partitions past it hold nothing of it
      const int np = my_pos[j] / p.partition_size + 1;
      if (part < np) store_head_t<D, BF16, true>(p, prow[j], part, np, phead[j], mq, o[j], m[j], lj);
    } else {
      store_head_t<D, BF16, false>(p, prow[j], 0, 1, phead[j], mq, o[j], m[j], lj);
    }
  }
}

template <int D, int PS, int W = kPrefillWaves>
static hipError_t launch_prefill_ps(const AttnParams& p, const int32_t* tiles, dim3 grid, bool bf16, bool kv8,
                                    hipStream_t stream) {
  const dim3 block(W * kWave);
  if (kv8) {
    if (bf16) hipLaunchKernelGGL((paged_prefill_kernel<D, true, true, PS, W>), grid, block, 0, stream, p, tiles);
    else hipLaunchKernelGGL((paged_prefill_kernel<D, false, true, PS, W>), grid, block, 0, stream, p, tiles);
  } else if (PS == 1 && bf16 && p.arrivals) {  // (for split tiles the second launch cost more than it saved)
    // the fp16 values pass, then the bf16 pass over the workgroups it handed back
    if constexpr (PS == 1) {
      hipLaunchKernelGGL((paged_prefill_kernel<D, true, false, PS, W, 1>), grid, block, 0, stream, p, tiles);
      hipLaunchKernelGGL((paged_prefill_kernel<D, true, false, PS, W, 2>), grid, block, 0, stream, p, tiles);
    }
  } else {
    if (bf16) hipLaunchKernelGGL((paged_prefill_kernel<D, true, false, PS, W>), grid, block, 0, stream, p, tiles);
    else hipLaunchKernelGGL((paged_prefill_kernel<D, false, false, PS, W>), grid, block, 0, stream, p, tiles);
  }
  return hipGetLastError();
}

// waves_per_group 1, 2, 4: tiles of the full capacity, a half, a quarter (4-wave workgroups);
// 0: the double tile (8-wave workgroups, head_dim 128 and 256).
template <int D>
static hipError_t launch_prefill_d(const AttnParams& p, const int32_t* tiles, dim3 grid, bool bf16, bool kv8,
                                   int waves_per_group, hipStream_t stream) {
  switch (waves_per_group) {
    case 0:
      if constexpr (D != 64) return launch_prefill_ps<D, 1, 8>(p, tiles, grid, bf16, kv8, stream);
      return hipErrorInvalidValue;
    case 1: return launch_prefill_ps<D, 1>(p, tiles, grid, bf16, kv8, stream);
    case 2: return launch_prefill_ps<D, 2>(p, tiles, grid, bf16, kv8, stream);
    case 4: return launch_prefill_ps<D, 4>(p, tiles, grid, bf16, kv8, stream);
    default: return hipErrorInvalidValue;
  }
}

int prefill_tile_pairs_for(int head_dim) {
  return (head_dim == 64 || head_dim == 128 || head_dim == 256) ? prefill_tile_pairs(head_dim) : 0;
}

hipError_t launch_prefill(const AttnParams& p, const int32_t* tiles, int n_tiles, int head_dim, bool bf16, bool kv8,
                          int waves_per_group, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)n_tiles * (p.num_heads / p.group)));
  switch (head_dim) {
    case 64: return launch_prefill_d<64>(p, tiles, grid, bf16, kv8, waves_per_group, stream);
    case 128: return launch_prefill_d<128>(p, tiles, grid, bf16, kv8, waves_per_group, stream);
    case 256: return launch_prefill_d<256>(p, tiles, grid, bf16, kv8, waves_per_group, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ayk
