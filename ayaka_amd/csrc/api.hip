// The C ABI of libayaka_hip (declared in include/ayaka_hip.h): argument
// checks, geometry, and the launches. No entry point allocates, frees or
// synchronises; all work is queued on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "ayaka_hip.h"
#include "ayaka_hip_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return AYK_OK;
}

int launched(hipError_t err, const char* what) {
  if (err != hipSuccess) return fail(AYK_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(err));
  return ok();
}

// The kernels' division of a position by the block size (block_of in attention_common.h):
// shift l = ceil(log2 bs) and magic m = floor(2^32 (2^l - bs) / bs) + 1, exact for every
// position below 2^31 (Granlund and Montgomery's round-up method; checked exhaustively on
// the host for every block size up to 300 and sampled ones up to 65536).
void block_divisor(int32_t bs, uint32_t& magic, int32_t& shift) {
  int s = 0;
  while ((1 << s) < bs) ++s;
  shift = s;
  magic = (uint32_t)(((uint64_t)1 << 32) * (((uint64_t)1 << s) - (uint64_t)bs) / (uint64_t)bs + 1);
}

// Split a group of query heads into equal chunks of at most 8 heads (one workgroup each).
int head_chunks_for(int group) {
  for (int n = 1; n <= group; ++n)
    if (group % n == 0 && group / n <= 8) return n;
  return group;
}

struct AttnCall {
  void* out;
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_table;
  int64_t table_stride;
  const int32_t* kv_lengths;
  const int32_t* request_of_row;
  const int32_t* positions;
  int32_t n_rows, num_heads, num_kv_heads, head_dim, num_blocks, block_size, max_blocks, layout,
      dtype, kv_dtype;
  float scale;
  float k_scale, v_scale;  // the cache holds keys / k_scale and values / v_scale (1, 1: as they are)
};

// Check a call and fill the launch record; returns AYK_OK or an error code.
int prepare(const char* op, const AttnCall& c, ayk::AttnParams& p, int& heads_per_chunk) {
  if (c.n_rows < 0) return fail(AYK_ERR_ARGUMENT, "%s: n_rows is negative (%d)", op, c.n_rows);
  if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
    return fail(AYK_ERR_UNSUPPORTED, "%s: head_dim %d is not one of 64, 128, 256", op, c.head_dim);
  if (c.dtype != AYK_DTYPE_FP16 && c.dtype != AYK_DTYPE_BF16 && c.dtype != AYK_DTYPE_FP32)
    return fail(AYK_ERR_UNSUPPORTED, "%s: dtype %d is not fp16 (0), bf16 (1) or fp32 (3)", op, c.dtype);
  if (c.kv_dtype != c.dtype && (c.kv_dtype != AYK_DTYPE_FP8_E4M3 || c.dtype == AYK_DTYPE_FP32))
    return fail(AYK_ERR_UNSUPPORTED, "%s: kv_dtype %d is neither the dtype (%d) nor fp8 e4m3 (2) under fp16/bf16", op,
                c.kv_dtype, c.dtype);
  if (c.layout != AYK_LAYOUT_NHD && c.layout != AYK_LAYOUT_HND)
    return fail(AYK_ERR_UNSUPPORTED, "%s: layout %d is not NHD (0) or HND (1)", op, c.layout);
  if (c.num_kv_heads <= 0 || c.num_heads <= 0 || c.num_heads % c.num_kv_heads != 0)
    return fail(AYK_ERR_ARGUMENT,
                "%s: %d query heads is not a positive multiple of %d key/value heads", op,
                c.num_heads, c.num_kv_heads);
  if (c.block_size < 1 || c.block_size > 65536)
    return fail(AYK_ERR_UNSUPPORTED, "%s: block_size %d is not in [1, 65536]", op, c.block_size);
  if (c.num_blocks <= 0 || c.max_blocks < 0 || c.table_stride < c.max_blocks)
    return fail(AYK_ERR_ARGUMENT, "%s: num_blocks %d, max_blocks %d, table_stride %lld", op,
                c.num_blocks, c.max_blocks, (long long)c.table_stride);
  if (c.max_blocks >= (1 << 24))
    return fail(AYK_ERR_UNSUPPORTED, "%s: a table of %d blocks per row exceeds 2^24", op, c.max_blocks);
  if ((c.request_of_row == nullptr) != (c.positions == nullptr))
    return fail(AYK_ERR_ARGUMENT, "%s: request_of_row and positions are given together or not at all",
                op);
  if (c.n_rows > 0 && (!c.out || !c.q || !c.k_cache || !c.v_cache || !c.block_table ||
                       !c.kv_lengths))
    return fail(AYK_ERR_ARGUMENT, "%s: a required pointer is null", op);
  const int group = c.num_heads / c.num_kv_heads;
  const int chunks = head_chunks_for(group);
  heads_per_chunk = group / chunks;
  p = ayk::AttnParams{};
  p.out = c.out;
  p.q = static_cast<const uint16_t*>(c.q);
  p.k_cache = static_cast<const uint16_t*>(c.k_cache);
  p.v_cache = static_cast<const uint16_t*>(c.v_cache);
  p.block_table = c.block_table;
  p.kv_lengths = c.kv_lengths;
  p.request_of_row = c.request_of_row;
  p.positions = c.positions;
  p.table_stride = c.table_stride;
  const int64_t D = c.head_dim, H = c.num_kv_heads, B = c.block_size;
  if (c.layout == AYK_LAYOUT_NHD) {
    p.block_stride = B * H * D;
    p.token_stride = H * D;
    p.head_stride = D;
  } else {
    p.block_stride = H * B * D;
    p.token_stride = D;
    p.head_stride = B * D;
  }
  if ((uint64_t)c.num_blocks * (uint64_t)p.block_stride > UINT32_MAX)
    return fail(AYK_ERR_UNSUPPORTED, "%s: a cache of %d blocks of %lld elements exceeds 32-bit element offsets",
                op, c.num_blocks, (long long)p.block_stride);
  if (p.token_stride >= (1 << 24))
    return fail(AYK_ERR_UNSUPPORTED, "%s: a token stride of %lld elements exceeds 2^24", op,
                (long long)p.token_stride);
  p.n_rows = c.n_rows;
  p.num_heads = c.num_heads;
  p.group = group;
  p.head_chunks = chunks;
  p.num_virtual_heads = c.num_kv_heads * chunks;
  p.num_blocks = c.num_blocks;
  p.block_size = c.block_size;
  block_divisor(c.block_size, p.bs_magic, p.bs_shift);
  // The kernels walk a context in 32-bit positions, a staged table segment (up to
  // kTableCap blocks) and a chunk past the current one at a time; a table whose positions
  // come within that reach of INT32_MAX could overflow those sums, so it is refused.
  const int64_t table_len = (int64_t)c.max_blocks * c.block_size;
  const int64_t max_table_len = INT32_MAX - (int64_t)(ayk::kTableCap + 1) * c.block_size - 4096;
  if (table_len > max_table_len)
    return fail(AYK_ERR_UNSUPPORTED, "%s: a table of %d blocks of %d positions exceeds %lld positions per row", op,
                c.max_blocks, c.block_size, (long long)max_table_len);
  p.max_len = (int32_t)table_len;
  if (!(c.k_scale > 0.f) || !(c.v_scale > 0.f) || !std::isfinite(c.k_scale) || !std::isfinite(c.v_scale))
    return fail(AYK_ERR_ARGUMENT, "%s: k_scale %g and v_scale %g must be positive and finite", op, c.k_scale,
                c.v_scale);
  // A key's score is scale * q.(k_scale * stored key): the key scale joins the score scale
  // (exact at k_scale 1), and a value's scale multiplies each normalised output.
  p.scale_log2 = c.scale * c.k_scale * 1.4426950408889634f;
  p.v_scale = c.v_scale;
  p.partition_size = INT32_MAX;
  p.max_partitions = 1;
  p.wave_split = 1;
  return AYK_OK;
}

// Compute units of the current device (queried once per device).
int compute_units() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Whether v2 merges its partitions inside the partition kernel (rather than in
// a reduce kernel) for a grid of `workgroups`. Measured on MI355X: the in-kernel
// merge costs each workgroup a device-scope release (an L2 write-back) and the
// last one of a row the merge; with the reduce kernel merging several heads per
// workgroup (a few hundred workgroups for C3) the second launch costs less on
// every benchmark grid (C3 161.4 vs 170.8 us, fp8 C5 228.0 vs 236.9, C5 a tie) but
// a tiny one: a grid of a few dozen workgroups is latency-bound, and there the
// second launch is the larger cost (C1 15.9 vs 18.9 us). The merging workgroup folds
// a row's partitions one round trip per two of them, so it only pays for rows of a
// few partitions: at one row of 2048 positions (32 x 4 heads of 64) the in-kernel
// merge over 32 partitions took 16.1 us per call in a graph replay, the reduce
// kernel 9.2; over 2-4 partitions the two sites measured within 0.1 us.
constexpr int kInKernelMaxPartitions = 4;
bool merge_in_kernel(int64_t workgroups, int max_partitions) {
  return workgroups <= compute_units() / 4 && max_partitions <= kInKernelMaxPartitions;
}

// Heads per wave from which the library picks the matrix-core q.k kernel.
constexpr int kMfmaMinHeads = 3;

constexpr int32_t kWaveFlags = AYK_FLAG_WAVES_1 | AYK_FLAG_WAVES_2 | AYK_FLAG_WAVES_4 | AYK_FLAG_WAVES_8;

// Waves that share one virtual head's positions: the AYK_FLAG_WAVES_* flag's count, else 1
// for v2 and, for v1, the most (up to 8) that keep rows x virtual heads x waves within one
// round of 8-wave workgroups on the GPU. A v1 workgroup per row covering every head (wave
// split 1) fills 64 of 256 compute units at C3's 64 rows; splitting each context among 4
// waves gives 256 workgroups of 2 heads.
int wave_split_for(const ayk::AttnParams& p, bool split, int32_t flags) {
  if (flags & AYK_FLAG_WAVES_1) return 1;
  if (flags & AYK_FLAG_WAVES_2) return 2;
  if (flags & AYK_FLAG_WAVES_4) return 4;
  if (flags & AYK_FLAG_WAVES_8) return 8;
  if (split) return 1;
  const int64_t slots = (int64_t)compute_units() * ayk::kMaxWavesPerGroup;
  int ws = 1;
  while (ws < ayk::kMaxWavesPerGroup && (int64_t)p.n_rows * p.num_virtual_heads * ws * 2 <= slots) ws *= 2;
  return ws;
}

// The q.k path and workgroup shape for a launch, then the kernel(s).
// fp32 models: the VALU decode kernel, one wave per virtual head, partitions merged by its own
// reduce kernel (no wave split, no single launch, no q.k choice).
int launch_f32(const char* op, const ayk::AttnParams& p, int head_dim, int gc, bool split, int32_t flags,
               void* stream) {
  if (flags & ~(AYK_FLAG_PARTIALS_ONLY | AYK_FLAG_SEPARATE_REDUCE | AYK_FLAG_WAVES_1))
    return fail(AYK_ERR_UNSUPPORTED, "%s: flags 0x%x: fp32 runs one kernel shape (partials only, a separate "
                "reduce and one wave per head are the flags it takes)", op, flags);
  ayk::AttnParams q = p;
  q.wave_split = 1;
  q.arrivals = nullptr;
  if (ayk::walking()) {  // the host address walk: the launch's loads, no launch
    ayk::walk_f32(q, head_dim, split);
    return ok();
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err = ayk::launch_attention_f32(q, head_dim, gc, split, s);
  if (err == hipSuccess && split && !(flags & AYK_FLAG_PARTIALS_ONLY))
    err = ayk::launch_partition_reduce_f32(q, head_dim, compute_units(), s);
  return launched(err, op);
}

int launch(const char* op, const ayk::AttnParams& p, int head_dim, int gc, bool bf16, bool kv8, bool split,
           int32_t flags, void* stream) {
  if (flags & ~(AYK_FLAG_QK_DPP | AYK_FLAG_QK_MFMA | AYK_FLAG_PARTIALS_ONLY | AYK_FLAG_SEPARATE_REDUCE |
                AYK_FLAG_SINGLE_LAUNCH | kWaveFlags))
    return fail(AYK_ERR_ARGUMENT, "%s: unknown flags 0x%x", op, flags);
  if (__builtin_popcount(flags & kWaveFlags) > 1)
    return fail(AYK_ERR_ARGUMENT, "%s: at most one AYK_FLAG_WAVES_* flag", op);
  if ((flags & AYK_FLAG_QK_DPP) && (flags & AYK_FLAG_QK_MFMA))
    return fail(AYK_ERR_ARGUMENT, "%s: AYK_FLAG_QK_DPP and AYK_FLAG_QK_MFMA exclude each other", op);
  if ((flags & AYK_FLAG_SEPARATE_REDUCE) && (flags & AYK_FLAG_SINGLE_LAUNCH))
    return fail(AYK_ERR_ARGUMENT, "%s: AYK_FLAG_SEPARATE_REDUCE and AYK_FLAG_SINGLE_LAUNCH exclude each other",
                op);
  if (kv8 && (flags & AYK_FLAG_QK_DPP))
    return fail(AYK_ERR_UNSUPPORTED, "%s: the DPP kernel reads 16-bit caches only, not fp8", op);
  // Measured on MI355X: from 3 heads per wave the matrix-core kernel (keys staged
  // through LDS) streams faster than the DPP kernel, whose per-token dot2 and
  // butterfly work grows with the group; 1-2 heads stay on the DPP kernel.
  // fp8 caches are read by the matrix-core kernel only.
  ayk::AttnParams q = p;
  // split each context (v1) or partition (v2) among waves of the matrix-core kernel (the DPP
  // kernel, forced, streams each head's positions in one wave)
  q.wave_split = (flags & AYK_FLAG_QK_DPP) ? 1 : wave_split_for(p, split, flags);
  if ((flags & AYK_FLAG_QK_DPP) && (flags & kWaveFlags) && !(flags & AYK_FLAG_WAVES_1))
    return fail(AYK_ERR_UNSUPPORTED, "%s: the DPP kernel does not split a context among waves", op);
  const bool mfma = kv8 || (flags & AYK_FLAG_QK_MFMA) || q.wave_split > 1 ||
                    (!(flags & AYK_FLAG_QK_DPP) && gc >= kMfmaMinHeads);
  const int waves = 4;
  const int64_t items = (split && p.work) ? p.n_work : (int64_t)p.n_rows * (split ? p.max_partitions : 1);
  const int64_t workgroups = items * p.num_virtual_heads;
  if (workgroups > INT32_MAX || (int64_t)p.n_rows * p.num_heads > INT32_MAX)
    return fail(AYK_ERR_UNSUPPORTED, "%s: %lld workgroups exceed one launch", op, (long long)workgroups);
  // The grid: one workgroup per item and group of up to kMaxWaves / wave_split virtual heads.
  const int heads_per_wg = ayk::kMaxWavesPerGroup / q.wave_split;
  const int64_t grid = items * ((p.num_virtual_heads + heads_per_wg - 1) / heads_per_wg);
  if (split && q.arrivals && !(flags & AYK_FLAG_SINGLE_LAUNCH) && !merge_in_kernel(grid, p.max_partitions))
    q.arrivals = nullptr;
  if (ayk::walking()) {  // the host address walk: the launch's loads, no launch
    ayk::walk_decode(q, head_dim, mfma, kv8, split, false);
    return ok();
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err = mfma ? ayk::launch_attention_mfma(q, head_dim, gc, bf16, split, kv8, waves, s)
                        : ayk::launch_attention_dpp(q, head_dim, gc, bf16, split, waves, s);
  if (err == hipSuccess && split && !q.arrivals && !(flags & AYK_FLAG_PARTIALS_ONLY))
    err = ayk::launch_partition_reduce(q, head_dim, bf16, compute_units(), s);
  return launched(err, op);
}

// Scratch of ayk_paged_attention_v2_static: one array per device, held until the process
// ends; partials (and their (m, l)) first, then the arrival counters, which are zero when
// the code object loads and which every call leaves at zero.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
constexpr size_t kStaticCounterWords = size_t(1) << 18;  // 1 MiB of uint32 counters at the end
constexpr size_t kStaticPartialBytes = kStaticScratchBytes - kStaticCounterWords * sizeof(uint32_t);
static_assert(kStaticPartialBytes == AYK_V2_STATIC_SCRATCH_BYTES, "the header states the partials' capacity");
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// The device address of `scratch` on the current device, looked up once per device
// (hipGetSymbolAddress with that device current); nullptr with an error set on failure.
// The array's name is a host-side stand-in: only this address may reach a kernel.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

void* static_scratch(const char* op, void* stream) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(AYK_ERR_LAUNCH, "%s: no current device (%s)", op, hipGetErrorString(err));
    return nullptr;
  }
  // The array is looked up on the current device; a stream of another device would run the
  // kernels there with this device's address, so the two must agree.
  if (stream) {
    int stream_dev = -1;
    err = hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_dev);
    if (err != hipSuccess) {
      fail(AYK_ERR_LAUNCH, "%s: hipStreamGetDevice: %s", op, hipGetErrorString(err));
      return nullptr;
    }
    if (stream_dev != dev) {
      fail(AYK_ERR_ARGUMENT, "%s: the stream belongs to device %d but device %d is current", op, stream_dev, dev);
      return nullptr;
    }
  }
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr) return ptr;
  err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (err != hipSuccess || !ptr) {
    fail(AYK_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", op, dev, hipGetErrorString(err));
    return nullptr;
  }
  g_scratch_ptr[dev].store(ptr, std::memory_order_release);  // two threads may race here: same address
  return ptr;
}

}  // namespace

extern "C" {

int ayk_abi_version(void) { return 18; }

int ayk_paged_prefill_tile_pairs(int32_t head_dim) { return ayk::prefill_tile_pairs_for(head_dim); }

const char* ayk_last_error(void) { return g_last_error.c_str(); }

int ayk_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                          const int64_t* slot_mapping, int64_t n_rows, int32_t num_kv_heads,
                          int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t layout,
                          int32_t elem_bytes, void* stream) {
  const char* op = "ayk_reshape_and_cache";
  if (n_rows < 0) return fail(AYK_ERR_ARGUMENT, "%s: n_rows is negative", op);
  if (num_kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0 || block_size <= 0)
    return fail(AYK_ERR_ARGUMENT, "%s: num_kv_heads %d, head_dim %d, num_blocks %d, block_size %d",
                op, num_kv_heads, head_dim, num_blocks, block_size);
  if (elem_bytes != 2 && elem_bytes != 4)
    return fail(AYK_ERR_UNSUPPORTED, "%s: elem_bytes %d is not 2 or 4", op, elem_bytes);
  if (layout != AYK_LAYOUT_NHD && layout != AYK_LAYOUT_HND)
    return fail(AYK_ERR_UNSUPPORTED, "%s: layout %d is not NHD (0) or HND (1)", op, layout);
  if (n_rows == 0) return ok();
  if (!k || !v || !k_cache || !v_cache || !slot_mapping)
    return fail(AYK_ERR_ARGUMENT, "%s: a required pointer is null", op);
  return launched(ayk::launch_reshape_and_cache(k, v, k_cache, v_cache, slot_mapping, n_rows,
                                                num_kv_heads, head_dim, num_blocks, block_size,
                                                layout == AYK_LAYOUT_HND, elem_bytes,
                                                static_cast<hipStream_t>(stream)),
                  op);
}

int ayk_reshape_and_cache_e4m3(const void* k, const void* v, void* k_cache, void* v_cache,
                               const int64_t* slot_mapping, int64_t n_rows, int32_t num_kv_heads, int32_t head_dim,
                               int32_t num_blocks, int32_t block_size, int32_t layout, int32_t src_dtype,
                               float k_scale, float v_scale, void* stream) {
  const char* op = "ayk_reshape_and_cache_e4m3";
  if (!(k_scale > 0.f) || !(v_scale > 0.f) || !std::isfinite(k_scale) || !std::isfinite(v_scale))
    return fail(AYK_ERR_ARGUMENT, "%s: k_scale %g and v_scale %g must be positive and finite", op, k_scale, v_scale);
  if (n_rows < 0) return fail(AYK_ERR_ARGUMENT, "%s: n_rows is negative", op);
  if (num_kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0 || block_size <= 0)
    return fail(AYK_ERR_ARGUMENT, "%s: num_kv_heads %d, head_dim %d, num_blocks %d, block_size %d",
                op, num_kv_heads, head_dim, num_blocks, block_size);
  if (src_dtype != AYK_DTYPE_FP16 && src_dtype != AYK_DTYPE_BF16)
    return fail(AYK_ERR_UNSUPPORTED, "%s: src_dtype %d is not fp16 (0) or bf16 (1)", op, src_dtype);
  if (layout != AYK_LAYOUT_NHD && layout != AYK_LAYOUT_HND)
    return fail(AYK_ERR_UNSUPPORTED, "%s: layout %d is not NHD (0) or HND (1)", op, layout);
  if (n_rows == 0) return ok();
  if (!k || !v || !k_cache || !v_cache || !slot_mapping)
    return fail(AYK_ERR_ARGUMENT, "%s: a required pointer is null", op);
  return launched(ayk::launch_reshape_and_cache_e4m3(k, v, k_cache, v_cache, slot_mapping, n_rows, num_kv_heads,
                                                     head_dim, num_blocks, block_size, layout == AYK_LAYOUT_HND,
                                                     src_dtype == AYK_DTYPE_BF16, 1.0f / k_scale, 1.0f / v_scale,
                                                     static_cast<hipStream_t>(stream)),
                  op);
}

int ayk_paged_attention_v1(void* out, const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* block_table, int64_t table_stride,
                           const int32_t* kv_lengths, const int32_t* request_of_row,
                           const int32_t* positions, int32_t n_rows, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                           int32_t block_size, int32_t max_blocks, int32_t layout, int32_t dtype,
                           int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t flags, void* stream) {
  const char* op = "ayk_paged_attention_v1";
  AttnCall c{out,       q,          k_cache,  v_cache,      block_table, table_stride,
             kv_lengths, request_of_row, positions, n_rows, num_heads, num_kv_heads,
             head_dim,  num_blocks, block_size, max_blocks, layout, dtype, kv_dtype, scale, k_scale, v_scale};
  ayk::AttnParams p;
  int gc = 0;
  const int rc = prepare(op, c, p, gc);
  if (rc != AYK_OK) return rc;
  if (n_rows == 0) return ok();
  if (dtype == AYK_DTYPE_FP32) return launch_f32(op, p, head_dim, gc, false, flags, stream);
  return launch(op, p, head_dim, gc, dtype == AYK_DTYPE_BF16, kv_dtype == AYK_DTYPE_FP8_E4M3, false, flags,
                stream);
}

size_t ayk_paged_attention_v2_workspace_bytes(int32_t n_rows, int32_t num_heads, int32_t head_dim,
                                              int32_t max_partitions) {
  if (n_rows <= 0 || num_heads <= 0 || head_dim <= 0 || max_partitions <= 0) return 0;
  const size_t parts = (size_t)n_rows * num_heads * max_partitions;
  // partial outputs first (16-byte aligned rows), then the (m, l) pairs
  return parts * (size_t)head_dim * sizeof(float) + parts * 2 * sizeof(float);
}

int ayk_paged_attention_v2(void* out, const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* block_table, int64_t table_stride,
                           const int32_t* kv_lengths, const int32_t* request_of_row,
                           const int32_t* positions, int32_t n_rows, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                           int32_t block_size, int32_t max_blocks, int32_t layout, int32_t dtype,
                           int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t partition_size, int32_t max_partitions,
                           const int32_t* work_items, int32_t n_work_items, const int32_t* staged,
                           void* workspace, size_t workspace_bytes, uint32_t* arrivals, int32_t flags,
                           void* stream) {
  const char* op = "ayk_paged_attention_v2";
  AttnCall c{out,       q,          k_cache,  v_cache,      block_table, table_stride,
             kv_lengths, request_of_row, positions, n_rows, num_heads, num_kv_heads,
             head_dim,  num_blocks, block_size, max_blocks, layout, dtype, kv_dtype, scale, k_scale, v_scale};
  ayk::AttnParams p;
  int gc = 0;
  const int rc = prepare(op, c, p, gc);
  if (rc != AYK_OK) return rc;
  if (partition_size <= 0 || partition_size % 64 != 0)
    return fail(AYK_ERR_ARGUMENT, "%s: partition_size %d is not a positive multiple of 64", op,
                partition_size);
  if (max_partitions <= 0 || max_partitions > 65535)
    return fail(AYK_ERR_ARGUMENT, "%s: max_partitions %d is not in [1, 65535]", op, max_partitions);
  if (n_work_items < 0 || (n_work_items > 0 && !work_items))
    return fail(AYK_ERR_ARGUMENT, "%s: %d work items at %p", op, n_work_items, (const void*)work_items);
  if (staged && n_work_items == 0)
    return fail(AYK_ERR_ARGUMENT, "%s: staged parameters need a work list (the grid's capacity)", op);
  if (n_rows == 0) return ok();
  // Staged parameters pack the rows' partials: at most one slot per work item.
  const int32_t slot_rows = staged ? n_work_items : n_rows;
  const int32_t slots_per_row = staged ? 1 : max_partitions;
  const size_t need = ayk_paged_attention_v2_workspace_bytes(slot_rows, num_heads, head_dim, slots_per_row);
  if (!workspace || workspace_bytes < need)
    return fail(AYK_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", op, workspace_bytes,
                need);
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(AYK_ERR_ARGUMENT, "%s: workspace is not 16-byte aligned", op);
  const size_t parts = (size_t)slot_rows * num_heads * slots_per_row;
  p.part_o = static_cast<float*>(workspace);
  p.part_ml = p.part_o + parts * head_dim;
  p.partition_size = partition_size;
  p.max_partitions = max_partitions;
  p.work = n_work_items > 0 ? work_items : nullptr;
  p.n_work = n_work_items;
  p.staged = staged;
  // The single launch merges in the partition kernel; without counters, or when
  // asked, a reduce kernel does (and PARTIALS_ONLY runs neither merge).
  p.arrivals = (flags & (AYK_FLAG_SEPARATE_REDUCE | AYK_FLAG_PARTIALS_ONLY)) ? nullptr : arrivals;
  p.max_len = (int32_t)std::min<int64_t>(p.max_len, (int64_t)partition_size * max_partitions);
  if (dtype == AYK_DTYPE_FP32) return launch_f32(op, p, head_dim, gc, true, flags, stream);
  return launch(op, p, head_dim, gc, dtype == AYK_DTYPE_BF16, kv_dtype == AYK_DTYPE_FP8_E4M3, true, flags,
                stream);
}

int ayk_paged_attention_v2_static(void* out, const void* q, const void* k_cache, const void* v_cache,
                                  const int32_t* block_table, int64_t table_stride, const int32_t* kv_lengths,
                                  const int32_t* request_of_row, const int32_t* positions, int32_t n_rows,
                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t num_blocks,
                                  int32_t block_size, int32_t max_blocks, int32_t layout, int32_t dtype,
                                  int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t partition_size, int32_t max_partitions,
                                  const int32_t* work_items, int32_t n_work_items, const int32_t* staged,
                                  int32_t flags, void* stream) {
  const char* op = "ayk_paged_attention_v2_static";
  const int32_t slot_rows = staged ? n_work_items : n_rows;
  const int32_t slots_per_row = staged ? 1 : max_partitions;
  const size_t need = ayk_paged_attention_v2_workspace_bytes(slot_rows, num_heads, head_dim, slots_per_row);
  if (need > kStaticPartialBytes)
    return fail(AYK_ERR_WORKSPACE,
                "%s: this call needs %zu bytes of scratch; the static scratch holds %zu (use ayk_paged_attention_v2 "
                "with a workspace)",
                op, need, kStaticPartialBytes);
  if (n_rows <= 0 || num_heads <= 0) {  // nothing to launch: the checks of the allocating entry point apply
    return ayk_paged_attention_v2(out, q, k_cache, v_cache, block_table, table_stride, kv_lengths, request_of_row,
                                  positions, n_rows, num_heads, num_kv_heads, head_dim, num_blocks, block_size,
                                  max_blocks, layout, dtype, kv_dtype, scale, k_scale, v_scale, partition_size, max_partitions,
                                  work_items, n_work_items, staged, nullptr, 0, nullptr, flags, stream);
  }
  unsigned char* base = static_cast<unsigned char*>(static_scratch(op, stream));
  if (!base) return AYK_ERR_LAUNCH;
  // counters for the single launch only when every (row, head) has one
  uint32_t* counters = (int64_t)n_rows * num_heads <= (int64_t)kStaticCounterWords
                           ? reinterpret_cast<uint32_t*>(base + kStaticPartialBytes)
                           : nullptr;
  return ayk_paged_attention_v2(out, q, k_cache, v_cache, block_table, table_stride, kv_lengths, request_of_row,
                                positions, n_rows, num_heads, num_kv_heads, head_dim, num_blocks, block_size,
                                max_blocks, layout, dtype, kv_dtype, scale, k_scale, v_scale, partition_size, max_partitions, work_items,
                                n_work_items, staged, base, kStaticPartialBytes, counters, flags, stream);
}

int ayk_paged_attention_v2_static_counters(void** counters, int64_t* words) {
  const char* op = "ayk_paged_attention_v2_static_counters";
  if (!counters || !words) return fail(AYK_ERR_ARGUMENT, "%s: a required pointer is null", op);
  unsigned char* base = static_cast<unsigned char*>(static_scratch(op, nullptr));
  if (!base) return AYK_ERR_LAUNCH;
  *counters = base + kStaticPartialBytes;
  *words = (int64_t)kStaticCounterWords;
  return ok();
}

int ayk_paged_prefill(void* out, const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* block_table, int64_t table_stride, const int32_t* kv_lengths,
                      const int32_t* request_of_row, const int32_t* positions, const int32_t* tiles,
                      int32_t n_tiles, int32_t tile_pairs, int32_t n_rows, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                      int32_t num_blocks, int32_t block_size, int32_t max_blocks, int32_t layout, int32_t dtype,
                      int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t partition_size, void* workspace,
                      size_t workspace_bytes, void* stream) {
  const char* op = "ayk_paged_prefill";
  if (!request_of_row || !positions)
    return fail(AYK_ERR_ARGUMENT, "%s: request_of_row and positions are required", op);
  AttnCall c{out,       q,          k_cache,  v_cache,      block_table, table_stride,
             kv_lengths, request_of_row, positions, n_rows, num_heads, num_kv_heads,
             head_dim,  num_blocks, block_size, max_blocks, layout,      dtype,       kv_dtype, scale, k_scale, v_scale};
  ayk::AttnParams p;
  int gc = 0;
  const int rc = prepare(op, c, p, gc);
  if (rc != AYK_OK) return rc;
  if (dtype == AYK_DTYPE_FP32)
    return fail(AYK_ERR_UNSUPPORTED, "%s: fp32 runs on the decode entry points, row by row", op);
  // Tiles of the full capacity, or of a half or a quarter (2 or 4 waves then share
  // each group of pairs and split its chunks), or at head_dim 128 and 256 of twice it (an
  // 8-wave workgroup; waves_per_group 0 below).
  const int full_pairs = ayk::prefill_tile_pairs_for(head_dim);
  const bool twice = head_dim != 64 && tile_pairs == 2 * full_pairs;
  const int waves_per_group = twice ? 0 : tile_pairs > 0 && full_pairs % tile_pairs == 0 ? full_pairs / tile_pairs : -1;
  if (waves_per_group != 0 && waves_per_group != 1 && waves_per_group != 2 && waves_per_group != 4)
    return fail(AYK_ERR_ARGUMENT, "%s: tile_pairs %d is not %d, %d or %d%s", op, tile_pairs, full_pairs,
                full_pairs / 2, full_pairs / 4, head_dim != 64 ? " (or twice the first)" : "");
  if (p.group > tile_pairs)
    return fail(AYK_ERR_UNSUPPORTED, "%s: %d query heads per key/value head exceed a tile of %d", op, p.group,
                tile_pairs);
  if (n_tiles < 0 || (n_tiles > 0 && !tiles))
    return fail(AYK_ERR_ARGUMENT, "%s: %d tiles at %p", op, n_tiles, (const void*)tiles);
  if ((int64_t)n_tiles * num_kv_heads > INT32_MAX)
    return fail(AYK_ERR_UNSUPPORTED, "%s: %d tiles x %d key/value heads exceed one launch", op, n_tiles,
                num_kv_heads);
  if (partition_size < 0 || partition_size % 64 != 0)
    return fail(AYK_ERR_ARGUMENT, "%s: partition_size %d is not 0 or a positive multiple of 64", op,
                partition_size);
  if (n_tiles == 0 || n_rows == 0) return ok();
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool walk = ayk::walking();  // the host address walk: the launch's loads, no launch
  // bf16 models over bf16 caches: a workspace with room for one int32 per workgroup (after the
  // partials, 16-byte aligned) lets the kernel run P.V in fp16 where the values allow and hand
  // the other workgroups to a bf16 pass (the slots need no initial contents)
  size_t partial_bytes = 0;
  if (partition_size > 0) {
    const int64_t parts = ((int64_t)p.max_len + partition_size - 1) / partition_size;
    if (parts >= 1 && parts <= 65535)
      partial_bytes = (ayk_paged_attention_v2_workspace_bytes(n_rows, num_heads, head_dim, (int32_t)parts) + 15) & ~size_t(15);
  }
  const size_t flag_bytes = (size_t)n_tiles * num_kv_heads * sizeof(uint32_t);
  if (dtype == AYK_DTYPE_BF16 && kv_dtype == AYK_DTYPE_BF16 && workspace && workspace_bytes >= partial_bytes + flag_bytes &&
      reinterpret_cast<uintptr_t>(workspace) % 16 == 0)
    p.arrivals = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + partial_bytes);
  if (partition_size == 0 && walk) {
    ayk::walk_prefill(p, tiles, n_tiles, head_dim, kv_dtype == AYK_DTYPE_FP8_E4M3, waves_per_group);
    return ok();
  }
  if (partition_size == 0)
    return launched(ayk::launch_prefill(p, tiles, n_tiles, head_dim, dtype == AYK_DTYPE_BF16,
                                        kv_dtype == AYK_DTYPE_FP8_E4M3, waves_per_group, s),
                    op);
  const int64_t max_partitions = ((int64_t)p.max_len + partition_size - 1) / partition_size;
  if (max_partitions < 1 || max_partitions > 65535)
    return fail(AYK_ERR_UNSUPPORTED, "%s: %lld partitions of %d positions per row are not in [1, 65535]", op,
                (long long)max_partitions, partition_size);
  const size_t need = ayk_paged_attention_v2_workspace_bytes(n_rows, num_heads, head_dim, (int32_t)max_partitions);
  if (!workspace || workspace_bytes < need)
    return fail(AYK_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", op, workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(AYK_ERR_ARGUMENT, "%s: workspace is not 16-byte aligned", op);
  const size_t parts = (size_t)n_rows * num_heads * max_partitions;
  p.part_o = static_cast<float*>(workspace);
  p.part_ml = p.part_o + parts * head_dim;
  p.partition_size = partition_size;
  p.max_partitions = (int32_t)max_partitions;
  if (walk) {
    ayk::walk_prefill(p, tiles, n_tiles, head_dim, kv_dtype == AYK_DTYPE_FP8_E4M3, waves_per_group);
    return ok();
  }
  hipError_t err = ayk::launch_prefill(p, tiles, n_tiles, head_dim, dtype == AYK_DTYPE_BF16,
                                       kv_dtype == AYK_DTYPE_FP8_E4M3, waves_per_group, s);
  if (err == hipSuccess) err = ayk::launch_row_reduce(p, head_dim, dtype == AYK_DTYPE_BF16, s);
  return launched(err, op);
}

int ayk_paged_attention_windows(void* out, const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* block_table, int64_t table_stride, const int32_t* kv_lengths,
                                const int32_t* request_of_row, const int32_t* positions, const int32_t* tiles,
                                int32_t n_tiles, int32_t n_rows, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t max_blocks,
                                int32_t layout, int32_t dtype, int32_t kv_dtype, float scale, float k_scale, float v_scale, int32_t partition_size,
                                void* workspace, size_t workspace_bytes, void* stream) {
  const char* op = "ayk_paged_attention_windows";
  if (!request_of_row || !positions)
    return fail(AYK_ERR_ARGUMENT, "%s: request_of_row and positions are required", op);
  AttnCall c{out,       q,          k_cache,  v_cache,      block_table, table_stride,
             kv_lengths, request_of_row, positions, n_rows, num_heads, num_kv_heads,
             head_dim,  num_blocks, block_size, max_blocks, layout,      dtype,       kv_dtype, scale, k_scale, v_scale};
  ayk::AttnParams p;
  int gc = 0;
  const int rc = prepare(op, c, p, gc);
  if (rc != AYK_OK) return rc;
  if (dtype == AYK_DTYPE_FP32)
    return fail(AYK_ERR_UNSUPPORTED, "%s: fp32 runs on the decode entry points, row by row", op);
  if (p.group > 16)
    return fail(AYK_ERR_UNSUPPORTED, "%s: %d query heads per key/value head exceed a window's 16 columns", op,
                p.group);
  if (n_tiles < 0 || (n_tiles > 0 && !tiles))
    return fail(AYK_ERR_ARGUMENT, "%s: %d tiles at %p", op, n_tiles, (const void*)tiles);
  if ((int64_t)n_tiles * num_kv_heads > INT32_MAX)
    return fail(AYK_ERR_UNSUPPORTED, "%s: %d tiles x %d key/value heads exceed one launch", op, n_tiles,
                num_kv_heads);
  if (partition_size < 0 || partition_size % 64 != 0)
    return fail(AYK_ERR_ARGUMENT, "%s: partition_size %d is not 0 or a positive multiple of 64", op,
                partition_size);
  if (n_tiles == 0 || n_rows == 0) return ok();
  // one wave per key/value head, its 16 columns the tile's (row, query head) pairs
  p.head_chunks = 1;
  p.num_virtual_heads = num_kv_heads;
  p.work = tiles;
  p.n_work = n_tiles;
  p.arrivals = nullptr;
  // Few tiles leave compute units idle: each key/value head of a tile then gets up to 8
  // waves, which take every n-th chunk and merge in LDS (as v1 does for decode rows),
  // the most that keep the launch within one round of 8-wave workgroups. Measured
  // (µs, one wave -> the chosen split, library partitions): 16 x 4-row windows over 1K
  // 33.8 -> 20.2, 32 x 4 over 4K 97.9 -> 89.7, 64 x 2 over 2K 89.2 -> 82.1.
  p.wave_split = 1;
  {
    const int64_t slots = (int64_t)compute_units() * ayk::kMaxWavesPerGroup;
    while (p.wave_split < ayk::kMaxWavesPerGroup && (int64_t)n_tiles * num_kv_heads * p.wave_split * 2 <= slots)
      p.wave_split *= 2;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == AYK_DTYPE_BF16, kv8 = kv_dtype == AYK_DTYPE_FP8_E4M3;
  const bool walk = ayk::walking();  // the host address walk: the launch's loads, no launch
  if (partition_size == 0 && walk) {
    ayk::walk_decode(p, head_dim, true, kv8, false, true);
    return ok();
  }
  if (partition_size == 0) return launched(ayk::launch_window_mfma(p, head_dim, bf16, false, kv8, s), op);
  const int64_t max_partitions = ((int64_t)p.max_len + partition_size - 1) / partition_size;
  if (max_partitions < 1 || max_partitions > 65535)
    return fail(AYK_ERR_UNSUPPORTED, "%s: %lld partitions of %d positions per row are not in [1, 65535]", op,
                (long long)max_partitions, partition_size);
  const size_t need = ayk_paged_attention_v2_workspace_bytes(n_rows, num_heads, head_dim, (int32_t)max_partitions);
  if (!workspace || workspace_bytes < need)
    return fail(AYK_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", op, workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(AYK_ERR_ARGUMENT, "%s: workspace is not 16-byte aligned", op);
  const size_t parts = (size_t)n_rows * num_heads * max_partitions;
  p.part_o = static_cast<float*>(workspace);
  p.part_ml = p.part_o + parts * head_dim;
  p.partition_size = partition_size;
  p.max_partitions = (int32_t)max_partitions;
  if (walk) {
    ayk::walk_decode(p, head_dim, true, kv8, true, true);
    return ok();
  }
  hipError_t err = ayk::launch_window_mfma(p, head_dim, bf16, true, kv8, s);
  if (err == hipSuccess) err = ayk::launch_row_reduce(p, head_dim, bf16, s);
  return launched(err, op);
}

static int block_op_checks(const char* op, int64_t n, int32_t num_blocks, int64_t block_bytes) {
  if (n < 0 || num_blocks <= 0 || block_bytes <= 0 || block_bytes % 2 != 0)
    return fail(AYK_ERR_ARGUMENT, "%s: n %lld, num_blocks %d, block_bytes %lld", op, (long long)n,
                num_blocks, (long long)block_bytes);
  if (n > INT32_MAX) return fail(AYK_ERR_ARGUMENT, "%s: too many blocks (%lld)", op, (long long)n);
  return AYK_OK;
}

int ayk_gather_blocks(const void* k_cache, const void* v_cache, void* out_k, void* out_v,
                      const void* block_ids, int32_t ids_are_64bit, int64_t n, int32_t num_blocks,
                      int64_t block_bytes, void* stream) {
  const char* op = "ayk_gather_blocks";
  const int rc = block_op_checks(op, n, num_blocks, block_bytes);
  if (rc != AYK_OK) return rc;
  if (n == 0) return ok();
  if (!k_cache || !v_cache || !out_k || !out_v || !block_ids)
    return fail(AYK_ERR_ARGUMENT, "%s: a required pointer is null", op);
  return launched(ayk::launch_block_op(0, k_cache, v_cache, out_k, out_v, block_ids, nullptr,
                                       ids_are_64bit != 0, n, num_blocks, block_bytes,
                                       static_cast<hipStream_t>(stream)),
                  op);
}

int ayk_copy_blocks(void* k_cache, void* v_cache, const void* src, const void* dst,
                    int32_t ids_are_64bit, int64_t n, int32_t num_blocks, int64_t block_bytes,
                    void* stream) {
  const char* op = "ayk_copy_blocks";
  const int rc = block_op_checks(op, n, num_blocks, block_bytes);
  if (rc != AYK_OK) return rc;
  if (n == 0) return ok();
  if (!k_cache || !v_cache || !src || !dst)
    return fail(AYK_ERR_ARGUMENT, "%s: a required pointer is null", op);
  return launched(ayk::launch_block_op(1, k_cache, v_cache, k_cache, v_cache, src, dst,
                                       ids_are_64bit != 0, n, num_blocks, block_bytes,
                                       static_cast<hipStream_t>(stream)),
                  op);
}

int ayk_zero_blocks(void* k_cache, void* v_cache, const void* block_ids, int32_t ids_are_64bit,
                    int64_t n, int32_t num_blocks, int64_t block_bytes, void* stream) {
  const char* op = "ayk_zero_blocks";
  const int rc = block_op_checks(op, n, num_blocks, block_bytes);
  if (rc != AYK_OK) return rc;
  if (n == 0) return ok();
  if (!k_cache || !v_cache || !block_ids)
    return fail(AYK_ERR_ARGUMENT, "%s: a required pointer is null", op);
  return launched(ayk::launch_block_op(2, nullptr, nullptr, k_cache, v_cache, block_ids, nullptr,
                                       ids_are_64bit != 0, n, num_blocks, block_bytes,
                                       static_cast<hipStream_t>(stream)),
                  op);
}

}  // extern "C"
