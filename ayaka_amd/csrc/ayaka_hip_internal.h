// Kernel parameter records and launchers shared by the HIP sources of libayaka_hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ayk {

// Most waves (one per virtual head) in one decode workgroup.
constexpr int kMaxWavesPerGroup = 8;
// Block-table entries staged in LDS per segment of a row's context.
constexpr int kTableCap = 512;

// Everything one paged-attention launch reads. Strides are in elements.
struct AttnParams {
  void* out;
  const uint16_t* q;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  const int32_t* block_table;
  const int32_t* kv_lengths;
  const int32_t* request_of_row;  // nullptr: row n is request n
  const int32_t* positions;       // nullptr: row n attends to its whole context
  const int32_t* work;            // v2 only, optional: n_work (row, partition) pairs to run
  const int32_t* staged;          // v2 only, optional (graph replays): {partition size, work items,
                                  // n_rows partial offsets} read on the device; the grid then covers
                                  // n_work items at most
  float* part_o;                  // v2 only: [n_rows, num_heads, max_partitions, head_dim], or with
                                  // staged parameters the rows packed (partial_index)
  float* part_ml;                 // v2 only: the same slots' (m, l)
  uint32_t* arrivals;             // v2 single launch: [n_rows, head groups] counters, zero between calls;
                                  // nullptr: a separate reduce kernel merges the partitions. Multi-row
                                  // kernel: one hand-off slot per workgroup for the fp16 values pass
                                  // (nullptr: one bf16 pass)
  int64_t table_stride;
  int64_t block_stride;
  int64_t token_stride;
  int64_t head_stride;
  int32_t n_rows;
  int32_t num_heads;
  int32_t group;        // query heads per key/value head
  int32_t head_chunks;  // chunks one group's heads are split into (group / head_chunks each)
  int32_t num_virtual_heads;  // num_kv_heads * head_chunks: the unit one wave serves
  int32_t num_blocks;
  int32_t block_size;
  uint32_t bs_magic;    // position t -> block (umulhi(t, bs_magic) + t) >> bs_shift, for any block
  int32_t bs_shift;     // size (a power of two: bs_magic 1, bs_shift its log2)
  int32_t max_len;      // no row reads positions at or past this
  int32_t partition_size;
  int32_t max_partitions;
  int32_t n_work;
  int32_t wave_split;   // v1, matrix-core kernel: waves sharing one virtual head's context
                        // (1, 2, 4 or 8; a workgroup holds 8 / wave_split virtual heads)
  float scale_log2;     // scale * k_scale * log2(e): scores live in the log2 domain
  float v_scale;        // each normalised output (and partial) is multiplied by it
};

// The per-(row, head[, partition]) attention kernels; `waves` is the workgroup size in waves.
hipError_t launch_attention_dpp(const AttnParams& p, int head_dim, int heads_per_chunk, bool bf16,
                                bool split, int waves, hipStream_t stream);
// kv8: the caches hold fp8 e4m3 codes (1 byte per element), decoded on load.
hipError_t launch_attention_mfma(const AttnParams& p, int head_dim, int heads_per_chunk, bool bf16,
                                 bool split, bool kv8, int waves, hipStream_t stream);
// Multi-row attention: one workgroup per (tile of rows of one request, key/value head).
// A tile holds at most prefill_tile_pairs_for(head_dim) (row, query head) pairs (0: unsupported).
int prefill_tile_pairs_for(int head_dim);
hipError_t launch_prefill(const AttnParams& p, const int32_t* tiles, int n_tiles, int head_dim, bool bf16, bool kv8,
                          int waves_per_group, hipStream_t stream);
// Window launch of the decode kernel: p.work holds p.n_work tiles of the multi-row tile list
// (first row, rows, request, partition) of at most 16 / group rows; p.head_chunks 1.
hipError_t launch_window_mfma(const AttnParams& p, int head_dim, bool bf16, bool split, bool kv8, hipStream_t stream);
// fp32 models: the VALU decode kernel (v1, or v2 partitions) and its partition merge.
hipError_t launch_attention_f32(const AttnParams& p, int head_dim, int heads_per_chunk, bool split,
                                hipStream_t stream);
hipError_t launch_partition_reduce_f32(const AttnParams& p, int head_dim, int compute_units, hipStream_t stream);
// The v2 log-sum-exp merge of the partitions of every (row, head); `compute_units` of the
// device sets how many partition slots each pair gets.
hipError_t launch_partition_reduce(const AttnParams& p, int head_dim, bool bf16, int compute_units,
                                   hipStream_t stream);
hipError_t launch_row_reduce(const AttnParams& p, int head_dim, bool bf16, hipStream_t stream);

// The host address walk (kv_reach.hip): while it is on for the calling thread, the attention
// entry points enumerate the K/V loads of the launch they prepared instead of launching it.
bool walking();
void walk_decode(const AttnParams& p, int head_dim, bool mfma, bool kv8, bool split, bool window);
void walk_f32(const AttnParams& p, int head_dim, bool split);
void walk_prefill(const AttnParams& p, const int32_t* tiles, int n_tiles, int head_dim, bool kv8,
                  int waves_per_group);

hipError_t launch_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                                    const int64_t* slot_mapping, int64_t n_rows, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t num_blocks, int32_t block_size,
                                    bool hnd, int32_t elem_bytes, hipStream_t stream);

// KV write into fp8 e4m3 caches from fp16 (bf16 = false) or bf16 rows.
// Each element is multiplied by its tensor's inverse scale (k_inv, v_inv) before it is encoded.
hipError_t launch_reshape_and_cache_e4m3(const void* k, const void* v, void* k_cache, void* v_cache,
                                         const int64_t* slot_mapping, int64_t n_rows, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t num_blocks, int32_t block_size, bool hnd,
                                         bool bf16, float k_inv, float v_inv, hipStream_t stream);

// mode: 0 = gather (dst index i), 1 = copy (dst ids), 2 = zero (no source)
hipError_t launch_block_op(int mode, const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                           const void* src_ids, const void* dst_ids, bool ids64, int64_t n,
                           int32_t num_blocks, int64_t block_bytes, hipStream_t stream);

}  // namespace ayk
