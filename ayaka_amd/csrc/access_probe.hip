// Read-only probes of the KV-cache access patterns a decode kernel can use.
//
// A measurement tool, not part of the library: each probe reads exactly the
// bytes one decode-attention call over the headline shape reads (64 rows x
// 4096 positions, 8 key/value heads, head_dim 128, bf16, blocks of 16 from a
// random permutation of 40000), with 128-bit loads, and does no arithmetic, so
// its time is the ceiling the pattern allows. Built by ayaka_amd._build into
// ayaka_amd/lib/access_probe; `python bench.py --access-probe` runs it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 64, kLen = 4096, kHeads = 8, kDim = 128, kBlock = 16, kPool = 40000;
constexpr int kBlocksPerRow = kLen / kBlock;

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                  \
      std::exit(1);                                                                \
    }                                                                              \
  } while (0)

template <bool NT>
__device__ __forceinline__ u32x4 load16(const uint16_t* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return *reinterpret_cast<const u32x4*>(p);
}

// Flat stream over one pool: U independent 16-byte loads per lane per step.
template <bool NT, int U = 4>
__global__ __launch_bounds__(256) void stream_probe(const uint16_t* src, size_t n16, uint32_t* sink) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * 256 * U;
  for (size_t base = (size_t)blockIdx.x * 256 * U + threadIdx.x; base < n16; base += stride) {
    u32x4 a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = base + (size_t)u * 256;
      a[u] = load16<NT>(src + (i < n16 ? i : 0) * 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= a[u].x ^ a[u].y ^ a[u].z ^ a[u].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

// Flat stream straight into LDS (global_load_lds, 16 bytes per lane): each wave fills its
// own 1 KB slice per load, 4 loads per step, and waits for them before the next step.
__global__ __launch_bounds__(256) void stream_lds_probe(const uint16_t* src, size_t n16, uint32_t* sink) {
  constexpr int U = 4;
  __shared__ u32x4 buf[4][U][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t stride = (size_t)gridDim.x * 256 * U;
  for (size_t base = (size_t)blockIdx.x * 256 * U + wave * 64 * U; base < n16; base += stride) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = base + (size_t)u * 64 + lane;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src + (i < n16 ? i : 0) * 8),
                                       (__attribute__((address_space(3))) void*)&buf[wave][u][0], 16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);
  }
  if (buf[wave][0][lane].x == 0x9e3779b9u) sink[0] = 1;
}

// Paged reads. A workgroup covers `part` positions of one row; HEADS_PER_WG
// heads are read by waves of the workgroup (1: the workgroup serves one head
// with 4 waves splitting the positions; 8: wave w serves head w). Lanes: 16 per
// position (256 contiguous bytes of one head), 4 positions per load, 2 loads
// per chunk of 8 positions for K and for V.
template <bool HND, int HEADS_PER_WG>
__global__ __launch_bounds__(512) void paged_probe(const uint16_t* k, const uint16_t* v, const int* table,
                                                   int part, uint32_t* sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int parts = kLen / part;
  int id = blockIdx.x;
  const int p = id % parts;
  id /= parts;
  int head, row, wave_step, first;
  if (HEADS_PER_WG == 1) {
    head = id % kHeads;
    row = id / kHeads;
    wave_step = 4;
    first = wave;
  } else {
    head = wave;
    row = id;
    wave_step = 1;
    first = 0;
  }
  const int* tbl = table + row * kBlocksPerRow;
  uint32_t acc = 0;
  for (int ci = first; ci < part / 8; ci += wave_step) {
    u32x4 a[4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = p * part + ci * 8 + j * 4 + lane / 16;
      const int blk = tbl[t / kBlock], off = t % kBlock;
      const size_t e = HND ? (((size_t)blk * kHeads + head) * kBlock + off) * kDim + (lane % 16) * 8
                           : (((size_t)blk * kBlock + off) * kHeads + head) * kDim + (lane % 16) * 8;
      a[j] = load16<true>(k + e);
      a[2 + j] = load16<true>(v + e);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc ^= a[j].x ^ a[j].y ^ a[j].z ^ a[j].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

template <typename F>
static float time_us(F launch) {
  for (int i = 0; i < 3; ++i) launch();
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  CHECK(hipEventRecord(a));
  const int reps = 20;
  for (int i = 0; i < reps; ++i) launch();
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return ms * 1000.f / reps;
}

int main() {
  const size_t elems = (size_t)kPool * kBlock * kHeads * kDim;
  uint16_t *k = nullptr, *v = nullptr;
  int* table = nullptr;
  uint32_t* sink = nullptr;
  CHECK(hipMalloc(&k, elems * 2));
  CHECK(hipMalloc(&v, elems * 2));
  CHECK(hipMalloc(&table, sizeof(int) * kRows * kBlocksPerRow));
  CHECK(hipMalloc(&sink, 4));
  CHECK(hipMemset(k, 1, elems * 2));
  CHECK(hipMemset(v, 1, elems * 2));
  std::vector<int> perm(kPool - 1);
  for (int i = 0; i < kPool - 1; ++i) perm[i] = i + 1;
  std::shuffle(perm.begin(), perm.end(), std::mt19937(1));
  CHECK(hipMemcpy(table, perm.data(), sizeof(int) * kRows * kBlocksPerRow, hipMemcpyHostToDevice));
  const double paged_bytes = (double)kRows * kLen * kHeads * kDim * 2 * 2;
  const double pool_bytes = (double)elems * 2 * 2;

  std::printf("%-58s %10s %10s\n", "pattern", "us", "GB/s");
  auto flat = [&](const char* name, auto kernel, int grid) {
    const float us = time_us([&] {
      kernel<<<grid, 256>>>(k, elems / 8, sink);
      kernel<<<grid, 256>>>(v, elems / 8, sink);
    });
    std::printf("%-58s %10.1f %10.0f\n", name, us, pool_bytes / us / 1e3);
  };
  flat("flat stream, plain loads", stream_probe<false>, 2048);
  flat("flat stream, nontemporal loads", stream_probe<true>, 2048);
  flat("flat stream, nontemporal, 8 loads per lane", stream_probe<true, 8>, 2048);
  flat("flat stream, nontemporal, 8 loads per lane, 8192 wgs", stream_probe<true, 8>, 8192);
  flat("flat stream, nontemporal, 16 loads per lane", stream_probe<true, 16>, 2048);
  flat("flat stream, straight to LDS (global_load_lds)", stream_lds_probe, 2048);
  struct Case {
    const char* name;
    bool hnd;
    int heads_per_wg;
    int part;
  };
  const Case cases[] = {
      {"NHD, wg per (row, head), whole context (4096)", false, 1, 4096},
      {"HND, wg per (row, head), whole context (4096)", true, 1, 4096},
      {"NHD, wg per (row, head, 512 positions)", false, 1, 512},
      {"HND, wg per (row, head, 512 positions)", true, 1, 512},
      {"NHD, wg per (row, 512 positions), wave per head", false, 8, 512},
      {"NHD, wg per (row, 1024 positions), wave per head", false, 8, 1024},
      {"HND, wg per (row, 512 positions), wave per head", true, 8, 512},
  };
  for (const Case& c : cases) {
    const int parts = kLen / c.part;
    const int wgs = kRows * parts * (c.heads_per_wg == 1 ? kHeads : 1);
    const int threads = c.heads_per_wg == 1 ? 256 : 512;
    const float us = time_us([&] {
      if (c.hnd) {
        if (c.heads_per_wg == 1) paged_probe<true, 1><<<wgs, threads>>>(k, v, table, c.part, sink);
        else paged_probe<true, 8><<<wgs, threads>>>(k, v, table, c.part, sink);
      } else {
        if (c.heads_per_wg == 1) paged_probe<false, 1><<<wgs, threads>>>(k, v, table, c.part, sink);
        else paged_probe<false, 8><<<wgs, threads>>>(k, v, table, c.part, sink);
      }
    });
    std::printf("%-58s %10.1f %10.0f\n", c.name, us, paged_bytes / us / 1e3);
  }
  CHECK(hipGetLastError());
  return 0;
}
