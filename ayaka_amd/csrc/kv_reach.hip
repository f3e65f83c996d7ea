// Host-side address walk of the attention kernels (no device code runs).
//
// With the walk on (ayk_debug_kv_reach_begin), the attention entry points check and prepare a
// launch exactly as usual -- the same strides, magic numbers, partition counts, wave split and
// work lists -- and then, instead of launching, enumerate on the host every K/V load the
// launch's workgroups would issue: the same loops as the kernels, the same chunk geometry and
// the same address arithmetic (kv_address.h), with the block table, lengths, positions and work
// list read from host memory. Each load's byte range relative to the cache base is folded into
// a reach [lo, hi); the table entries staged are checked against the table's extent too. A CPU
// test then asserts that every launch of every kernel, codec, head width and block size stays
// inside the cache it was given. The staged table segment sits between guard entries whose
// offsets point far past any cache, so an index outside the staged segment shows in the reach.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <vector>

#include "ayaka_hip.h"
#include "ayaka_hip_internal.h"
#include "kv_address.h"

namespace ayk {

namespace {

struct Walk {
  bool on = false;
  int64_t table_entries = 0;  // int32 entries of the block-table allocation
  int64_t lo = INT64_MAX, hi = INT64_MIN, loads = 0;
  int64_t table_lo = INT64_MAX, table_hi = INT64_MIN;
};

thread_local Walk g_walk;

constexpr uint32_t kGuard = 0xF0000000u;  // the offset a guard entry yields: far past any cache

void record(int64_t byte, int bytes) {
  g_walk.lo = std::min(g_walk.lo, byte);
  g_walk.hi = std::max(g_walk.hi, byte + bytes);
  ++g_walk.loads;
}

// The staged segment [s0, s1) of a request's table, as stage_table leaves it in LDS, with guard
// entries on both sides; returns the first staged block index.
int stage(const AttnParams& p, int64_t table_row, int s0, int s1, std::vector<uint32_t>& buffer) {
  const int b0 = block_of(p, s0);
  const int nb = block_of(p, s1 - 1) - b0 + 1;
  buffer.assign(3 * kTableCap, kGuard);
  for (int i = 0; i < nb; ++i) {
    const int64_t at = table_row + b0 + i;
    g_walk.table_lo = std::min(g_walk.table_lo, at);
    g_walk.table_hi = std::max(g_walk.table_hi, at + 1);
    const int32_t id = (at >= 0 && at < g_walk.table_entries) ? p.block_table[at] : -1;
    if (i < kTableCap) buffer[kTableCap + i] = table_entry(p, id);
  }
  if (nb > kTableCap) g_walk.table_hi = std::max<int64_t>(g_walk.table_hi, INT64_MAX / 2);  // over capacity
  return b0;
}

// row_context of the kernels, on host memory.
void row_of(const AttnParams& p, int row, int& req, int& len) {
  req = p.request_of_row ? p.request_of_row[row] : row;
  len = p.kv_lengths[req];
  if (len > 0 && p.positions) len = imin(len, p.positions[row] + 1);
  len = imax(0, imin(len, p.max_len));
}

struct Item {
  int row, part;
};

// The (row, partition) items a decode launch's workgroups cover.
std::vector<Item> decode_items(const AttnParams& p, bool split) {
  std::vector<Item> items;
  if (split && p.work) {
    const int n = p.staged ? std::min(p.n_work, p.staged[1]) : p.n_work;
    for (int i = 0; i < n; ++i) items.push_back(Item{p.work[2 * i], p.work[2 * i + 1]});
  } else {
    for (int r = 0; r < p.n_rows; ++r)
      for (int part = 0; part < (split ? p.max_partitions : 1); ++part) items.push_back(Item{r, part});
  }
  return items;
}

// Bytes of element `elem` of a cache and of one load: KV8 1-byte codes (8-byte loads), or
// 16-bit elements (16-byte loads); the fp32 kernel's 4-byte elements (16-byte loads) use
// F32Elems.
template <bool KV8>
struct KvElems {
  static int64_t bytes(int64_t elem) { return kv_bytes_of<KV8>(elem); }
  static constexpr int load = kv_load_bytes<KV8>();
  static constexpr int per_lane = 8;  // elements a lane's piece covers
};
template <int F>
struct F32Elems {  // F floats per lane, read as F / 4 adjacent 16-byte loads: one 4F-byte range
  static int64_t bytes(int64_t elem) { return 4 * elem; }
  static constexpr int load = 4 * F;
  static constexpr int per_lane = F;
};

// The loads of one wave of a decode launch (the matrix-core kernel, its window launch, the
// DPP kernel or the fp32 kernel): positions [t_begin, t_end) of request req, this wave's chunks
// of each segment.
template <class E>
void walk_wave(const AttnParams& p, int req, int t_begin, int t_end, int kvh, int slice, int ws, int ch, int tpl,
               int cpt, int loads_per_chunk, bool prefetch_clamped, std::vector<uint32_t>& buffer) {
  const int seg_len = segment_positions(p, ch);
  const uint32_t token_stride = (uint32_t)p.token_stride;
  for (int s0 = t_begin; s0 < t_end; s0 += seg_len) {
    const int s1 = imin(t_end, s0 + seg_len);
    const int b0 = stage(p, (int64_t)req * p.table_stride, s0, s1, buffer);
    const int nch = (s1 - s0 + ch - 1) / ch;
    if (slice >= nch) continue;
    const int last = prefetch_clamped ? last_chunk_of_slice(nch, slice, ws) : nch - 1;
    for (int ci = slice; ci <= last; ci += ws)
      for (int lane = 0; lane < 64; ++lane) {
        const int r = lane / cpt, c = lane % cpt;
        for (int j = 0; j < loads_per_chunk; ++j) {
          const uint32_t off = kv_offset(p, buffer.data() + kTableCap, b0, chunk_position(s0, s1, ci, ch, j, tpl, r),
                                         token_stride);
          record(E::bytes((int64_t)kvh * p.head_stride + c * E::per_lane + (int64_t)off), E::load);
        }
      }
  }
}

template <int D, bool KV8>
void walk_mfma(const AttnParams& p, bool split) {
  constexpr int CH = decode_tile_positions() * decode_tiles_per_chunk(D, KV8);
  constexpr int TPL = positions_per_load(D);
  std::vector<uint32_t> buffer;
  const int ws = p.wave_split;
  const int heads = std::min(p.num_virtual_heads, kMaxWavesPerGroup / ws);
  const int groups = (p.num_virtual_heads + heads - 1) / heads;
  for (const Item& it : decode_items(p, split))
    for (int g = 0; g < groups; ++g)
      for (int wave = 0; wave < heads * ws; ++wave) {
        const int vh = g * heads + wave / ws;
        if (vh >= p.num_virtual_heads) continue;
        int req, len;
        row_of(p, it.row, req, len);
        int t_begin = 0, t_end = len;
        if (split) {
          const int psize = p.staged ? p.staged[0] : p.partition_size;
          t_begin = it.part * psize;
          t_end = imin(len, t_begin + psize);
        }
        walk_wave<KvElems<KV8>>(p, req, t_begin, t_end, vh / p.head_chunks, wave % ws, ws, CH, TPL,
                                pieces_per_position(D), CH / TPL, true, buffer);
      }
}

template <int D, bool KV8>
void walk_window(const AttnParams& p, bool split) {
  constexpr int CH = decode_tile_positions() * decode_tiles_per_chunk(D, KV8);
  constexpr int TPL = positions_per_load(D);
  std::vector<uint32_t> buffer;
  const int ws = p.wave_split;
  const int heads = std::min(p.num_virtual_heads, kMaxWavesPerGroup / ws);
  const int groups = (p.num_virtual_heads + heads - 1) / heads;
  for (int item = 0; item < p.n_work; ++item) {
    const int first = p.work[4 * item], rows = p.work[4 * item + 1], req = p.work[4 * item + 2],
              part = p.work[4 * item + 3];
    int len = imax(0, imin(p.kv_lengths[req], p.max_len));
    if (len > 0) len = imax(0, imin(len, p.positions[first + rows - 1] + 1));
    if (len == 0) continue;
    int t_begin = 0, t_end = len;
    if (split) {
      t_begin = part * p.partition_size;
      if (t_begin >= len) continue;
      t_end = imin(len, t_begin + p.partition_size);
    }
    for (int g = 0; g < groups; ++g)
      for (int wave = 0; wave < heads * ws; ++wave) {
        const int vh = g * heads + wave / ws;
        if (vh >= p.num_virtual_heads) continue;
        walk_wave<KvElems<KV8>>(p, req, t_begin, t_end, vh, wave % ws, ws, CH, TPL, pieces_per_position(D),
                                CH / TPL, true, buffer);
      }
  }
}

template <int D>
void walk_dpp(const AttnParams& p, bool split) {
  constexpr int TPL = positions_per_load(D);
  constexpr int CH = TPL * dpp_loads_per_chunk();
  std::vector<uint32_t> buffer;
  for (const Item& it : decode_items(p, split))
    for (int vh = 0; vh < p.num_virtual_heads; ++vh) {
      int req, len;
      row_of(p, it.row, req, len);
      int t_begin = 0, t_end = len;
      if (split) {
        const int psize = p.staged ? p.staged[0] : p.partition_size;
        t_begin = it.part * psize;
        t_end = imin(len, t_begin + psize);
      }
      walk_wave<KvElems<false>>(p, req, t_begin, t_end, vh / p.head_chunks, 0, 1, CH, TPL, pieces_per_position(D),
                                dpp_loads_per_chunk(), false, buffer);
    }
}

template <int D, int GC>
void walk_f32_d(const AttnParams& p, bool split) {
  constexpr int F = f32_floats_per_lane(GC);
  constexpr int LPT = f32_lanes_per_position(D, GC);
  constexpr int TPL = 64 / LPT;
  constexpr int CH = TPL * f32_loads_per_chunk(GC);
  std::vector<uint32_t> buffer;
  for (const Item& it : decode_items(p, split))
    for (int vh = 0; vh < p.num_virtual_heads; ++vh) {
      int req, len;
      row_of(p, it.row, req, len);
      int t_begin = 0, t_end = len;
      if (split) {
        const int psize = p.staged ? p.staged[0] : p.partition_size;
        t_begin = it.part * psize;
        t_end = imin(len, t_begin + psize);
      }
      walk_wave<F32Elems<F>>(p, req, t_begin, t_end, vh / p.head_chunks, 0, 1, CH, TPL, LPT, f32_loads_per_chunk(GC),
                          false, buffer);
    }
}

template <int D, bool KV8, int PS, int N, int THREADS>
void walk_prefill_typed(const AttnParams& p, const int32_t* tiles, int n_tiles) {
  constexpr int CH = prefill_chunk_positions(D, PS);
  constexpr int CPT = pieces_per_position(D);
  static_assert(CH * CPT == N * THREADS, "a chunk's pieces, N per thread");
  const int tile_pairs = prefill_tile_pairs_for(D) * (THREADS / 256) / PS;
  const int kv_heads = p.num_heads / p.group;
  const uint32_t token_stride = (uint32_t)p.token_stride;
  std::vector<uint32_t> buffer;
  const bool split = p.part_o != nullptr;
  for (int tile = 0; tile < n_tiles; ++tile) {
    const int first_row = tiles[4 * tile], req = tiles[4 * tile + 2];
    const int part = split ? tiles[4 * tile + 3] : 0;
    const int n_pairs = std::min(tiles[4 * tile + 1] * p.group, tile_pairs);
    const int n_rows = (n_pairs + p.group - 1) / p.group;
    const int kv_len = imax(0, imin(p.kv_lengths[req], p.max_len));
    if (kv_len == 0) continue;
    const int last_pos = imin(p.positions[first_row + n_rows - 1], kv_len - 1);
    const int t_begin = split ? part * p.partition_size : 0;
    const int t_end = split ? imin(last_pos + 1, t_begin + p.partition_size) : last_pos + 1;
    const int seg_len = segment_positions(p, CH);
    for (int kvh = 0; kvh < kv_heads; ++kvh)
      for (int s0 = t_begin; s0 < t_end; s0 += seg_len) {
        const int s1 = imin(t_end, s0 + seg_len);
        const int b0 = stage(p, (int64_t)req * p.table_stride, s0, s1, buffer);
        const int nch = (s1 - s0 + CH - 1) / CH;
        for (int ci = 0; ci < nch; ++ci)
          for (int tid = 0; tid < THREADS; ++tid) {
            uint32_t off[N];
            prefill_offsets<N>(p, buffer.data() + kTableCap, b0, s0 + ci * CH + N * (tid / CPT), s1, tid % CPT,
                               token_stride, off);
            for (int u = 0; u < N; ++u)
              record(kv_bytes_of<KV8>((int64_t)kvh * p.head_stride + (int64_t)off[u]), kv_load_bytes<KV8>());
          }
      }
  }
}

template <int D, bool KV8, int PS, int THREADS = 256>
void walk_prefill_ps(const AttnParams& p, const int32_t* tiles, int n_tiles) {
  constexpr int N = prefill_chunk_positions(D, PS) * pieces_per_position(D) / THREADS;
  walk_prefill_typed<D, KV8, PS, N, THREADS>(p, tiles, n_tiles);
}

template <int D, bool KV8>
void walk_prefill_d(const AttnParams& p, const int32_t* tiles, int n_tiles, int waves_per_group) {
  switch (waves_per_group) {
    case 0:  // the double tile: 8-wave workgroups (head_dim 128 and 256)
      if constexpr (D != 64) walk_prefill_ps<D, KV8, 1, 512>(p, tiles, n_tiles);
      break;
    case 1: walk_prefill_ps<D, KV8, 1>(p, tiles, n_tiles); break;
    case 2: walk_prefill_ps<D, KV8, 2>(p, tiles, n_tiles); break;
    default: walk_prefill_ps<D, KV8, 4>(p, tiles, n_tiles); break;
  }
}

template <int D>
void walk_decode_d(const AttnParams& p, bool mfma, bool kv8, bool split, bool window) {
  if (window) return kv8 ? walk_window<D, true>(p, split) : walk_window<D, false>(p, split);
  if (!mfma) return walk_dpp<D>(p, split);
  return kv8 ? walk_mfma<D, true>(p, split) : walk_mfma<D, false>(p, split);
}

}  // namespace

bool walking() { return g_walk.on; }

void walk_decode(const AttnParams& p, int head_dim, bool mfma, bool kv8, bool split, bool window) {
  switch (head_dim) {
    case 64: walk_decode_d<64>(p, mfma, kv8, split, window); break;
    case 128: walk_decode_d<128>(p, mfma, kv8, split, window); break;
    default: walk_decode_d<256>(p, mfma, kv8, split, window); break;
  }
}

template <int GC>
void walk_f32_gc(const AttnParams& p, int head_dim, bool split) {
  switch (head_dim) {
    case 64: walk_f32_d<64, GC>(p, split); break;
    case 128: walk_f32_d<128, GC>(p, split); break;
    default: walk_f32_d<256, GC>(p, split); break;
  }
}

void walk_f32(const AttnParams& p, int head_dim, bool split) {
  // the kernel's lane geometry depends only on whether its heads per wave take the wide rows
  if (f32_floats_per_lane(p.group / p.head_chunks) == 8) walk_f32_gc<8>(p, head_dim, split);
  else walk_f32_gc<1>(p, head_dim, split);
}

void walk_prefill(const AttnParams& p, const int32_t* tiles, int n_tiles, int head_dim, bool kv8,
                  int waves_per_group) {
  switch (head_dim) {
    case 64:
      return kv8 ? walk_prefill_d<64, true>(p, tiles, n_tiles, waves_per_group)
                 : walk_prefill_d<64, false>(p, tiles, n_tiles, waves_per_group);
    case 128:
      return kv8 ? walk_prefill_d<128, true>(p, tiles, n_tiles, waves_per_group)
                 : walk_prefill_d<128, false>(p, tiles, n_tiles, waves_per_group);
    default:
      return kv8 ? walk_prefill_d<256, true>(p, tiles, n_tiles, waves_per_group)
                 : walk_prefill_d<256, false>(p, tiles, n_tiles, waves_per_group);
  }
}

}  // namespace ayk

extern "C" {

int ayk_debug_kv_reach_begin(int64_t table_entries) {
  if (table_entries < 0) return AYK_ERR_ARGUMENT;
  ayk::g_walk = ayk::Walk{};
  ayk::g_walk.on = true;
  ayk::g_walk.table_entries = table_entries;
  return AYK_OK;
}

int ayk_debug_kv_reach_end(int64_t* reach) {
  if (!reach) return AYK_ERR_ARGUMENT;
  const ayk::Walk w = ayk::g_walk;
  ayk::g_walk = ayk::Walk{};
  reach[0] = w.loads ? w.lo : 0;
  reach[1] = w.loads ? w.hi : 0;
  reach[2] = w.loads;
  reach[3] = w.table_hi >= w.table_lo ? w.table_lo : 0;
  reach[4] = w.table_hi >= w.table_lo ? w.table_hi : 0;
  return AYK_OK;
}

}  // extern "C"
