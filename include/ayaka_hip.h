/*
 * ayaka_hip.h -- C ABI of the MI355X (gfx950) paged-attention decode path.
 *
 * Every entry point is a plain C function over raw device pointers, sizes and a
 * hipStream_t passed as `void*`. None of them allocates, frees or synchronises:
 * the caller owns every buffer (the v2 scratch included) and the work is queued
 * asynchronously on `stream`. Each returns AYK_OK (0) or an AYK_ERR_* code; the
 * message of the last failure on the calling thread is ayk_last_error().
 *
 * The layouts are the ones Ayaka's ops contract defines
 * (reference python/ayaka/ops/kvcache.py:8-38):
 *   NHD cache: [num_blocks, block_size, num_kv_heads, head_dim], contiguous
 *   HND cache: [num_blocks, num_kv_heads, block_size, head_dim], contiguous
 *   slot = block_id * block_size + offset; block 0 is the padding block.
 *   q / out:   [n_rows, num_heads, head_dim], contiguous
 *   block table: int32 [n_requests, table_stride], row b lists request b's blocks.
 * Query head h reads key/value head h / (num_heads / num_kv_heads).
 *
 * Ids are not range-checked against the caller's intent (reference
 * python/ayaka/ops/kvcache.py:97-100), but nothing here reads or writes out of
 * bounds on bad metadata: block ids are clamped into [0, num_blocks), lengths
 * into the table width, and store drops rows whose slot is outside the pool.
 */
#ifndef AYAKA_HIP_H
#define AYAKA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  AYK_OK = 0,
  AYK_ERR_ARGUMENT = 1,    /* a size, pointer or combination the call cannot serve */
  AYK_ERR_UNSUPPORTED = 2, /* a head width / dtype / layout no kernel is built for */
  AYK_ERR_LAUNCH = 3,      /* the HIP runtime refused the launch */
  AYK_ERR_WORKSPACE = 4    /* the v2 workspace is smaller than ayk_paged_attention_v2_workspace_bytes */
};

/* Element types. fp16/bf16 for q, out and 16-bit caches; AYK_DTYPE_FP8_E4M3 for
 * caches of the "fp8_e4m3" codec: OCP fp8 e4m3 codes (torch.float8_e4m3fn), 1
 * byte per element, decoded exactly to the compute dtype when read; AYK_DTYPE_FP32
 * for fp32 models (q, out and caches all fp32; decode entry points only, on the VALU:
 * ayk_paged_attention_v1 / _v2 / _v2_static, whose rows may carry positions, so a
 * multi-row step runs row by row; the window and multi-row entry points refuse it). */
enum { AYK_DTYPE_FP16 = 0, AYK_DTYPE_BF16 = 1, AYK_DTYPE_FP8_E4M3 = 2, AYK_DTYPE_FP32 = 3 };

/* flags of the attention calls: 0 lets the library pick the q.k path. */
enum {
  AYK_FLAG_QK_DPP = 1,  /* q.k on the VALU: v_dot2 + DPP butterflies */
  AYK_FLAG_QK_MFMA = 2, /* q.k on the matrix cores: v_mfma_f32_16x16x32 */
  AYK_FLAG_PARTIALS_ONLY = 4, /* v2: run only the partition kernel (rows of several partitions are not
                                 written); for timing it */
  AYK_FLAG_SEPARATE_REDUCE = 8, /* v2: merge partitions in a second kernel even when arrivals is given */
  AYK_FLAG_SINGLE_LAUNCH = 16,  /* v2: merge partitions in the partition kernel (needs arrivals) */
  /* how many waves share each (row, key/value head)'s context (v1) or partition (v2), each
   * streaming every n-th 16-position chunk, their states merged in LDS at the end (at most
   * one of these; none lets the library pick: 1 for v2, and for v1 the most, up to 8, that
   * keep rows x heads x waves within one round of the GPU) */
  AYK_FLAG_WAVES_1 = 32,
  AYK_FLAG_WAVES_2 = 64,
  AYK_FLAG_WAVES_4 = 128,
  AYK_FLAG_WAVES_8 = 256
};
enum { AYK_LAYOUT_NHD = 0, AYK_LAYOUT_HND = 1 };

/* Version of this ABI; bumped on any signature change. */
int ayk_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ayk_last_error(void);

/*
 * KV write ("reshape_and_cache"): row i of k and v ([n_rows, num_kv_heads,
 * head_dim], contiguous, elem_bytes per element) is copied bit for bit into
 * slot slot_mapping[i] of k_cache and v_cache. Replaces the reference's
 * KVCacheOps.store, python/ayaka/ops/backends/torch/kvcache.py:65-80
 * (an index_put by slot). Padding rows carry slot 0 and all land in block 0.
 */
int ayk_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                          const int64_t* slot_mapping, int64_t n_rows, int32_t num_kv_heads,
                          int32_t head_dim, int32_t num_blocks, int32_t block_size,
                          int32_t layout, int32_t elem_bytes, void* stream);

/*
 * KV write into caches of the "fp8_e4m3" codec: row i of k and v (fp16 or bf16
 * per src_dtype, [n_rows, num_kv_heads, head_dim], contiguous) is encoded to
 * fp8 e4m3 codes and written to slot slot_mapping[i] (1 byte per element).
 * Encoding rounds to nearest even; a magnitude that rounds above 448, and NaN,
 * give the NaN code (no saturation), exactly as torch's cast to float8_e4m3fn.
 * The reference defines the codec field and only the "raw" codec
 * (python/ayaka/ops/kvcache.py:35-36, :54-55); this is KVCacheOps.store
 * (python/ayaka/ops/backends/torch/kvcache.py:65-80) for a quantised one.
 * k_scale and v_scale (positive, finite; 1 for none) are the layer's scales: an
 * element x is stored as the code of x * (1 / scale), the inverse rounded once to
 * fp32 and the product rounded once to fp32 before the encoding, so a cache of
 * keys up to 448 * k_scale stays finite. The attention entry points take the same
 * scales and read code * scale.
 */
int ayk_reshape_and_cache_e4m3(const void* k, const void* v, void* k_cache, void* v_cache,
                               const int64_t* slot_mapping, int64_t n_rows, int32_t num_kv_heads, int32_t head_dim,
                               int32_t num_blocks, int32_t block_size, int32_t layout, int32_t src_dtype,
                               float k_scale, float v_scale,
                               void* stream);

/*
 * Paged attention, single pass ("v1"): every page of a row's context is streamed
 * once per key/value head, in one launch and with no scratch. A workgroup serves
 * one row and 8 / n of its key/value heads, n waves per head (n = 1, 2, 4 or 8, see
 * AYK_FLAG_WAVES_*): each wave streams every n-th 16-position chunk and serves
 * the head's query heads from it, and the waves' states are merged in LDS, in wave
 * order. So the grid has rows x heads x n / 8 workgroups: C3's 64 rows fill the
 * GPU's 256 compute units with n = 4. Replaces the reference's decode attention,
 * python/ayaka/ops/backends/torch/attention.py:237-271 (_attend_decode), and
 * the row-causal multi-row path of the same file, :209-234.
 *
 * Rows: with request_of_row == NULL and positions == NULL, row i is request i
 * and attends to positions [0, kv_lengths[i]) (a decode step). Otherwise row i
 * belongs to request request_of_row[i] and attends to [0, positions[i] + 1)
 * (reference python/ayaka/ops/attention.py:12-30). A row whose request has
 * kv_lengths 0 is a padding row and gets zeros. Scores are scale * q.k in fp32,
 * the softmax and the value sum are fp32, and out is rounded once.
 * head_dim must be 64, 128 or 256 and block_size in [1, 65536]. `dtype` is
 * the type of q and out; `kv_dtype` that of the caches: the same, or
 * AYK_DTYPE_FP8_E4M3 (decoded exactly to `dtype` as it is read; matrix-core
 * kernel only). k_scale and v_scale (positive, finite; 1 for an unscaled cache,
 * which leaves every result bit as without them) say the cache holds keys / k_scale
 * and values / v_scale: a score is scale * k_scale * q.k over the stored keys (one
 * fp32 product for the two scales) and each normalised output is multiplied by
 * v_scale before rounding. The other attention entry points take them the same way.
 * `flags` (AYK_FLAG_QK_*) forces one q.k implementation; 0 picks by group size
 * (matrix cores from 3 query heads per key/value head).
 */
int ayk_paged_attention_v1(void* out, const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* block_table, int64_t table_stride,
                           const int32_t* kv_lengths, const int32_t* request_of_row,
                           const int32_t* positions, int32_t n_rows, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                           int32_t block_size, int32_t max_blocks, int32_t layout, int32_t dtype,
                           int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t flags,
                           void* stream);

/* Bytes of scratch ayk_paged_attention_v2 needs for these sizes. */
size_t ayk_paged_attention_v2_workspace_bytes(int32_t n_rows, int32_t num_heads, int32_t head_dim,
                                              int32_t max_partitions);

/*
 * Paged attention, split context ("v2"): one workgroup per (row, key/value
 * head, partition of partition_size positions) writes a partial result and its
 * log-sum-exp state into `workspace`; the partitions of each (row, head) are
 * then merged and rounded once. A row whose context fits one partition skips
 * the scratch and is rounded exactly as v1 rounds it.
 *
 * With `arrivals` (n_rows * num_heads uint32 words, all zero before the first
 * call that uses them) the merge can happen in the same launch: the workgroup
 * that finishes a row's partitions last merges them, and leaves its counter at
 * zero again, so the buffer stays ready for the next call. It must not be
 * shared by calls that overlap in time. The library takes the single launch
 * for a tiny grid (a quarter of the GPU's compute units at most), and a second
 * (reduce) kernel otherwise; AYK_FLAG_SINGLE_LAUNCH and
 * AYK_FLAG_SEPARATE_REDUCE force one. With NULL arrivals the reduce kernel
 * merges. Either way the merge folds the partitions in partition order,
 * so results do not depend on scheduling. Same arguments and semantics
 * as v1, plus the partition size (a positive multiple of 64) and the number of
 * partitions per row the scratch holds: every row's length must be at most
 * max_partitions * partition_size (positions beyond it are not read).
 * work_items, if not NULL, lists n_work_items (row, partition) int32 pairs --
 * the partitions that hold tokens, in the order to run them (longest first
 * balances best); partitions not listed are not computed, so the list must
 * cover every partition below ceil(length / partition_size) of every row,
 * each once (the arrival count relies on it), and partition 0 of every row
 * with no context (that workgroup writes the row's zeros). With
 * NULL the grid covers every (row, partition < max_partitions). staged, if not
 * NULL, is device memory holding 2 + n_rows int32, {partition size, item count,
 * then each row's first partial slot}, that the kernels read when they run, with
 * work_items then read up to that count: a graph replay follows the split and the
 * work list a host wrote for its step. The staged size is a multiple of 64 of at
 * least partition_size (which max_partitions covers); n_work_items is then the
 * list's capacity, which sizes the grid, and the staged count must not exceed it;
 * workgroups past the count return at once. Row r's partials take the slots from
 * its staged offset on, one per partition that holds tokens (offsets: a prefix sum
 * of ceil(length / size) over the rows), and the workspace holds n_work_items
 * slots: ayk_paged_attention_v2_workspace_bytes(n_work_items, num_heads, head_dim, 1).
 * The math the reference delegates to flashinfer's split-KV decode and its plan-time schedule
 * (python/ayaka/ops/backends/flashinfer/attention.py:221-251, :326).
 */
int ayk_paged_attention_v2(void* out, const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* block_table, int64_t table_stride,
                           const int32_t* kv_lengths, const int32_t* request_of_row,
                           const int32_t* positions, int32_t n_rows, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                           int32_t block_size, int32_t max_blocks, int32_t layout, int32_t dtype,
                           int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t partition_size,
                           int32_t max_partitions,
                           const int32_t* work_items, int32_t n_work_items, const int32_t* staged,
                           void* workspace, size_t workspace_bytes, uint32_t* arrivals, int32_t flags,
                           void* stream);

/*
 * ayk_paged_attention_v2 for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference:
 * the same arguments, semantics and kernels as ayk_paged_attention_v2 without `workspace`,
 * `workspace_bytes` and `arrivals`. The partials live in a static device array of the
 * library, a code-object global of 64 MiB: it is allocated on each device when the library's
 * code object loads there (the runtime loads it on a device's first use by this library,
 * whichever entry point that is), and held until the process ends, whether or not this entry
 * point is ever called. An engine's memory ledger should count it as memory a library takes
 * on its own (the reference's `runtime` owner, python/ayaka/memory/budget.py:43-48). It holds
 * AYK_V2_STATIC_SCRATCH_BYTES of partials, then 2^18 arrival counters, zero when the code
 * object loads and left at zero by every call. A call whose partials need more (see
 * ayk_paged_attention_v2_workspace_bytes) is refused with AYK_ERR_WORKSPACE; one of more
 * than 2^18 (row, head) pairs merges in the reduce kernel. Nothing is allocated, freed or
 * synchronised. The array is the current device's: `stream` must belong to the current device
 * (a stream of another device is refused with AYK_ERR_ARGUMENT). Every call on a device
 * shares that device's array: calls that overlap in time on one device (other streams, other
 * threads) race, and must be serialised by the caller.
 */
#define AYK_V2_STATIC_SCRATCH_BYTES ((size_t)63 << 20)
int ayk_paged_attention_v2_static(void* out, const void* q, const void* k_cache, const void* v_cache,
                                  const int32_t* block_table, int64_t table_stride, const int32_t* kv_lengths,
                                  const int32_t* request_of_row, const int32_t* positions, int32_t n_rows,
                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                                  int32_t block_size, int32_t max_blocks, int32_t layout, int32_t dtype,
                                  int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t partition_size,
                           int32_t max_partitions,
                                  const int32_t* work_items, int32_t n_work_items, const int32_t* staged,
                                  int32_t flags, void* stream);

/*
 * Diagnostic, no counterpart in the reference: the current device's address of the arrival
 * counters of ayk_paged_attention_v2_static (`*counters`, uint32 words) and their number
 * (`*words`), so a test can read them back and check that every call left them at zero.
 * Looks the array up as the entry point does; launches, allocates and synchronises nothing.
 */
int ayk_paged_attention_v2_static_counters(void** counters, int64_t* words);

/*
 * Multi-row paged attention (prefill chunks, verify windows): the rows of each
 * request are its last rows, row i at position positions[i] attends to
 * [0, positions[i]] of its request's context; rows of a request with
 * kv_lengths 0 get zeros. tiles lists n_tiles (first_row, row_count, request,
 * partition) int32 quadruples: consecutive rows of one request with row_count *
 * (num_heads / num_kv_heads) <= tile_pairs, covering every row once (rows past
 * that many pairs are not computed). tile_pairs is
 * ayk_paged_prefill_tile_pairs(head_dim), or a half or a quarter of it: smaller
 * tiles (few rows per request, verify windows) share each tile's chunks among 2
 * or 4 waves instead of spending them on empty pairs. At head_dim 128 and 256 it
 * may also be twice that capacity: the tile then runs in an 8-wave workgroup,
 * one per compute unit, which stages each chunk once for all its pairs. One workgroup per
 * (tile, key/value head) loads each chunk of the context once into LDS for all
 * its rows and query heads; q.k and P.V run on the matrix cores with fp32
 * accumulation. With partition_size 0 a tile covers its whole context and its
 * partition field must be 0. With a positive partition_size (a multiple of 64),
 * a tile entry covers positions [partition * partition_size, +partition_size)
 * of its rows' context, and the tiles must list, for every group of rows, each
 * partition below ceil((last row's position + 1) / partition_size) once; the
 * partitions store partials in workspace (at least
 * ayk_paged_attention_v2_workspace_bytes(n_rows, num_heads, head_dim,
 * ceil(max_blocks * block_size / partition_size)) bytes, 16-byte aligned) and
 * a reduce kernel on the same stream merges them, each row over its own
 * partitions in partition order. Small launches (few rows per request, verify
 * windows) fill the GPU this way. Replaces the reference's per-request SDPA loop,
 * python/ayaka/ops/backends/torch/attention.py:209-234, and flashinfer's batch
 * prefill (python/ayaka/ops/backends/flashinfer/attention.py:150-152, :253-266).
 * bf16 models over bf16 caches: a workspace with room, after the partials (16-byte
 * aligned), for one int32 per workgroup (n_tiles * num_kv_heads) lets the kernel stage
 * each chunk's values as fp16 and run P.V in one fp16 MFMA where all of a chunk's values
 * are fp16 values (|v| < 65536, at least one of them 2^-10 or more; values below 2^-17 round
 * to within 2^-25), and hand every other workgroup to a second, bf16 pass; the slots need no
 * initial contents. Without that room every workgroup runs the bf16 P.V.
 */
/* (row, query head) pairs one tile of ayk_paged_prefill may hold: 128 for head_dim
 * 64 and 128, 64 for 256, 0 for a width with no kernel. No reference counterpart: it
 * sizes the tiles the caller builds.
 */
int ayk_paged_prefill_tile_pairs(int32_t head_dim);

int ayk_paged_prefill(void* out, const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* block_table, int64_t table_stride, const int32_t* kv_lengths,
                      const int32_t* request_of_row, const int32_t* positions, const int32_t* tiles,
                      int32_t n_tiles, int32_t tile_pairs, int32_t n_rows, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                      int32_t num_blocks, int32_t block_size, int32_t max_blocks, int32_t layout, int32_t dtype,
                      int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t partition_size, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Attention for rows of few per request (verify windows, short chunks), on the decode
 * kernel: each tile of the multi-row tile list (int32 quadruples (first row, rows,
 * request, partition), as for ayk_paged_prefill, with at most 16 / (num_heads /
 * num_kv_heads) rows each) is one work item; a wave serves one key/value head and its
 * 16 matrix-core columns are the tile's (row, query head) pairs, each row masked at its
 * own position, so a request's context is streamed once for all the tile's rows. When
 * tiles x key/value heads leave compute units idle, the library gives each head up to 8
 * waves that split its chunks and merge in LDS (the most that keep the launch within one
 * round of 8-wave workgroups).
 * The rows of a tile are consecutive rows of one request whose positions rise (the
 * tile's last row sees the most: nothing past its position is read); a row whose position
 * is negative sees nothing and gets zeros. partition_size 0 covers each tile's context in
 * one workgroup; otherwise tiles carry partitions of that size (a multiple of 64) and the
 * rows spanning several are merged as in ayk_paged_prefill (same workspace). The multi-row
 * rule of the reference
 * (python/ayaka/ops/backends/torch/attention.py:209-234), as ayk_paged_prefill.
 */
int ayk_paged_attention_windows(void* out, const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* block_table, int64_t table_stride, const int32_t* kv_lengths,
                                const int32_t* request_of_row, const int32_t* positions, const int32_t* tiles,
                                int32_t n_tiles, int32_t n_rows, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t max_blocks,
                                int32_t layout, int32_t dtype, int32_t kv_dtype, float scale, float k_scale, float v_scale,
                                int32_t partition_size,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Whole-block copies of both caches; block_bytes is the size of one block of
 * one cache (block_size * num_kv_heads * head_dim * elem_bytes), the same in
 * either layout. Ids are int64 when ids_are_64bit, else int32.
 *
 * ayk_gather_blocks: out_k[i] = k_cache[block_ids[i]] (and v), for i < n.
 *   Replaces python/ayaka/ops/backends/torch/kvcache.py:83-93 (gather).
 * ayk_copy_blocks: block dst[i] = block src[i] in both caches.
 *   Replaces python/ayaka/ops/backends/torch/kvcache.py:96-107 (copy_blocks).
 * ayk_zero_blocks: every byte of the listed blocks set to zero.
 *   Replaces python/ayaka/ops/backends/torch/kvcache.py:110-115 (zero_blocks).
 */
int ayk_gather_blocks(const void* k_cache, const void* v_cache, void* out_k, void* out_v,
                      const void* block_ids, int32_t ids_are_64bit, int64_t n, int32_t num_blocks,
                      int64_t block_bytes, void* stream);
int ayk_copy_blocks(void* k_cache, void* v_cache, const void* src, const void* dst,
                    int32_t ids_are_64bit, int64_t n, int32_t num_blocks, int64_t block_bytes,
                    void* stream);
int ayk_zero_blocks(void* k_cache, void* v_cache, const void* block_ids, int32_t ids_are_64bit,
                    int64_t n, int32_t num_blocks, int64_t block_bytes, void* stream);

/*
 * Host-side launch model (no device work; callable without a GPU). No counterpart in the
 * reference, whose split-KV scheduling happens inside flashinfer's plan
 * (python/ayaka/ops/backends/flashinfer/attention.py:221-251).
 *
 * ayk_split_model: for each of `n_sizes` partition sizes, the modelled finish time (in
 * positions) of a v2 launch over the rows' `lengths` (rows of length <= 0 hold no work): each
 * row split into partitions of the size, the work items ordered longest first, each repeated
 * `groups` times (workgroups per item), dealt to XCD i mod `xcds`, each XCD handing its next
 * item to whichever of its `compute_units / xcds` units frees first, an item costing its
 * positions plus `cost`. Writes `makespans[c]` and, if `item_counts` is not null, the work
 * items per group at each size. Returns AYK_OK, or AYK_ERR_ARGUMENT for bad sizes or pointers.
 *
 * ayk_work_list: the v2 work list of rows of `lengths` at `partition_size`, as int32
 * (row, partition) pairs into `out` (2 words per item): full partitions by row then partition,
 * then each row's partial last partition, longest first (ties by row), then partition 0 of
 * every row without context. Returns the item count (with `out` null: the count only), or -1
 * for bad arguments.
 */
int ayk_split_model(const int64_t* lengths, int32_t n_lengths, const int32_t* sizes, int32_t n_sizes,
                    int32_t groups, int32_t cost, int32_t compute_units, int32_t xcds, int64_t* makespans,
                    int64_t* item_counts);
int64_t ayk_work_list(const int64_t* lengths, int32_t n_lengths, int32_t partition_size, int32_t* out);
/*
 * ayk_best_split: the index (`*best`) of the candidate size with the smallest
 * ayk_split_model finish time (the first of equal ones), among those with at most `max_items`
 * work items when `max_items` > 0 (-1 if none has), leaving out those whose items x `groups`
 * exceed `round_items` unless it is the last such candidate. Only candidates whose lower bound
 * can still beat the best found are scheduled in full.
 */
int ayk_best_split(const int64_t* lengths, int32_t n_lengths, const int32_t* sizes, int32_t n_sizes, int32_t groups,
                   int32_t cost, int32_t compute_units, int32_t xcds, int64_t max_items, int64_t round_items,
                   int32_t* best);
/*
 * ayk_dispatch_makespan: the finish time (`*makespan`) of `n` workgroups of these durations
 * started longest first, each in the first of `slots` identical slots to free up (the
 * multi-row launch model: a slot per workgroup a compute unit holds). Returns AYK_OK, or
 * AYK_ERR_ARGUMENT for a negative count, no slot or a null pointer.
 */
int ayk_dispatch_makespan(const double* durations, int64_t n, int32_t slots, double* makespan);

/*
 * Diagnostics, no counterpart in the reference: the host address walk. Between
 * ayk_debug_kv_reach_begin and ayk_debug_kv_reach_end on one thread, the attention entry
 * points (ayk_paged_attention_v1 / _v2 / _windows, ayk_paged_prefill) check and prepare each
 * call as usual but launch nothing: they enumerate on the host every K/V load its workgroups
 * would issue, with the kernels' own loops and address arithmetic. For the walk, the block
 * table, lengths, request_of_row, positions, work list, staged split and tiles arguments are
 * HOST pointers, and the q / out / cache / workspace pointers are never dereferenced.
 * `table_entries` is the int32 entry count of the table allocation. ayk_debug_kv_reach_end
 * writes reach[0..4]: the lowest byte and one past the highest byte any load touches, relative
 * to a cache's base (K and V share their offsets), the number of loads, and the range
 * [reach[3], reach[4]) of table entries read; then it turns the walk off. Needs no GPU.
 */
int ayk_debug_kv_reach_begin(int64_t table_entries);
int ayk_debug_kv_reach_end(int64_t* reach);

#ifdef __cplusplus
}
#endif

#endif /* AYAKA_HIP_H */
