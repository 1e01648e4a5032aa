// Read-only HBM probes for the paged-attention decode's practical ceiling on MI355X (gfx950).
//
// No attention math: each kernel only loads and folds the loaded words into one XOR per lane, so
// its time is what the memory system allows for that access pattern, launch size and number of
// loads in flight.  Two patterns:
//
//   stream  G workgroups of 256 threads; workgroup w reads its own contiguous span of the launch's
//           bytes, 16 bytes per lane per load, with U loads per lane in flight (a rolling window).
//   paged   the decode's access pattern: one workgroup per (sequence, KV head, partition) job reads
//           the K and V rows (head_dim 128, 16-bit: 256 bytes per token and head) of its partition's
//           tokens through a shuffled block table (16-token blocks, 8 KV heads, so a token's rows
//           of all heads are adjacent, as in the [num_blocks, block_size, kv_heads, head_dim]
//           layout).  Each wave reads 4 tokens per load instruction (one row per 16 lanes), K and V
//           together, U of each in flight.  The job's block ids are staged in LDS first, as the
//           decode stages its block-table slice.  `xcd` places all heads of a (sequence,
//           partition) on one XCD, the decode's placement for large grids.
//
// The reads come from HBM: a small launch reads a region the preceding launches did not (a rotation
// over 1 GiB, four times the 256 MB last-level cache), and a large one reads 4 GiB or more.  Output: one
// JSON object per configuration with microseconds per launch (HIP events around back-to-back
// launches, launch gaps included) and GB/s over the bytes read.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <random>
#include <vector>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                          \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                                       \
    }                                                                                     \
  } while (0)

namespace {

constexpr int kThreads = 256;
constexpr int kRowBytes = 256;       // one token's row of one KV head (head_dim 128, 16-bit)
constexpr int kBlockTokens = 16;
constexpr int kMaxJobBlocks = 256;   // block ids staged per job (partition <= 4096 tokens)

__device__ __forceinline__ uint32_t fold(u32x4 x) { return x[0] ^ x[1] ^ x[2] ^ x[3]; }

// n16: 16-byte units per workgroup; (n16 / 256) loads per lane, a multiple of U (host-checked).
template <int U>
__global__ __launch_bounds__(kThreads) void stream_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const u32x4* base = src + static_cast<int64_t>(blockIdx.x) * n16 + threadIdx.x;
  const int64_t n = n16 / kThreads;
  u32x4 r[U];
#pragma unroll
  for (int i = 0; i < U; ++i) r[i] = __builtin_nontemporal_load(base + i * kThreads);
  uint32_t acc = 0;
  for (int64_t k = U; k < n; k += U) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      acc ^= fold(r[i]);
      r[i] = __builtin_nontemporal_load(base + (k + i) * kThreads);
    }
  }
#pragma unroll
  for (int i = 0; i < U; ++i) acc ^= fold(r[i]);
  if (acc == 0x9e3779b9u) sink[blockIdx.x * kThreads + threadIdx.x] = acc;  // keeps the loads live
}

struct PagedArgs {
  const unsigned char* k;
  const unsigned char* v;
  const int* table;  // [seqs, blocks_per_seq] block ids of this region
  int seqs, heads, blocks_per_seq, part_tokens, parts;
  int64_t row_stride, block_stride;  // bytes
  int xcd;
};

// One job per workgroup; its partition's tokens split over 4 waves, 16 tokens per round.
template <int U>
__global__ __launch_bounds__(kThreads) void paged_kernel(PagedArgs a, uint32_t* __restrict__ sink) {
  __shared__ int s_blocks[kMaxJobBlocks];
  const int64_t hw = blockIdx.x;
  int64_t job = hw;
  if (a.xcd) {  // heads of one (sequence, partition) on XCD hw % 8; grid is a multiple of 8 * heads
    const int64_t row = hw / 8;
    job = ((row / a.heads) * 8 + hw % 8) * a.heads + row % a.heads;
  }
  const int head = static_cast<int>(job % a.heads);
  const int64_t rest = job / a.heads;
  const int seq = static_cast<int>(rest % a.seqs);
  const int part = static_cast<int>(rest / a.seqs);
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 4, j = lane & 15;
  const int job_blocks = a.part_tokens / kBlockTokens;
  const int first_block = part * job_blocks;
  for (int i = tid; i < job_blocks; i += kThreads)
    s_blocks[i] = a.table[static_cast<int64_t>(seq) * a.blocks_per_seq + first_block + i];
  __syncthreads();
  // Round i covers tokens 16 i .. 16 i + 15 of the partition (block i of the job); this lane's token
  // in it is 4 * wave + g.  Block-relative offset of this lane's 16 bytes:
  const int64_t lane_off = (4 * wave + g) * a.row_stride + static_cast<int64_t>(head) * kRowBytes + j * 16;
  const int n = job_blocks;  // rounds; a multiple of U (host-checked)
  auto offset = [&](int i) -> int64_t {
    const int blk = __builtin_amdgcn_readfirstlane(s_blocks[i]);
    return static_cast<int64_t>(blk) * a.block_stride + lane_off;
  };
  u32x4 rk[U], rv[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const int64_t off = offset(i);
    rk[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.k + off));
    rv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.v + off));
  }
  uint32_t acc = 0;
  for (int i0 = U; i0 < n; i0 += U) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      acc ^= fold(rk[i]) ^ fold(rv[i]);
      const int64_t off = offset(i0 + i);
      rk[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.k + off));
      rv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.v + off));
    }
  }
#pragma unroll
  for (int i = 0; i < U; ++i) acc ^= fold(rk[i]) ^ fold(rv[i]);
  if (acc == 0x9e3779b9u) sink[blockIdx.x * kThreads + tid] = acc;
}

struct Timer {
  hipEvent_t a, b;
  Timer() {
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
  }
  ~Timer() {
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
  }
};

// Microseconds per launch of launch(i) over `iters` back-to-back launches after a warmup.
template <class F>
double time_launches(F launch, int iters) {
  Timer t;
  for (int i = 0; i < std::max(20, iters / 4); ++i) launch(i);
  CHECK(hipDeviceSynchronize());
  CHECK(hipEventRecord(t.a));
  for (int i = 0; i < iters; ++i) launch(i);
  CHECK(hipEventRecord(t.b));
  CHECK(hipEventSynchronize(t.b));
  float ms = 0.0f;
  CHECK(hipEventElapsedTime(&ms, t.a, t.b));
  return ms * 1e3 / iters;
}

int iterations_for(int64_t bytes) {  // about 100 GB read per configuration, 20 to 3000 launches
  return static_cast<int>(std::max<int64_t>(20, std::min<int64_t>(3000, int64_t{100000000000} / bytes)));
}

template <int U>
void stream_case(const unsigned char* pool, int64_t pool_bytes, uint32_t* sink, int64_t sink_words, int groups,
                 int64_t launch_bytes) {
  const int64_t n16 = launch_bytes / groups / 16;
  if (launch_bytes % (int64_t{groups} * 16 * kThreads) != 0 || (n16 / kThreads) % U != 0 || n16 / kThreads < U ||
      int64_t{groups} * kThreads > sink_words) {
    std::fprintf(stderr, "stream: unsupported size (groups %d, bytes %lld, U %d)\n", groups,
                 static_cast<long long>(launch_bytes), U);
    std::exit(2);
  }
  const int64_t regions = pool_bytes / launch_bytes;
  if (regions < 1) std::exit(2);
  const u32x4* base = reinterpret_cast<const u32x4*>(pool);
  const int64_t region16 = launch_bytes / 16;
  const double us = time_launches(
      [&](int i) { stream_kernel<U><<<groups, kThreads>>>(base + (i % regions) * region16, n16, sink); },
      iterations_for(launch_bytes));
  std::printf("{\"pattern\": \"stream\", \"bytes\": %lld, \"workgroups\": %d, \"loads_in_flight\": %d, "
              "\"us\": %.2f, \"GBps\": %.0f}\n",
              static_cast<long long>(launch_bytes), groups, U, us, launch_bytes / (us * 1e3));
  std::fflush(stdout);
}

struct PagedShape {
  const char* name;
  int seqs, tokens, part_tokens, xcd;
};

template <int U>
void paged_case(unsigned char* pool, int64_t pool_bytes, uint32_t* sink, int64_t sink_words, const PagedShape& s) {
  constexpr int kHeads = 8;
  const int64_t row_stride = int64_t{kHeads} * kRowBytes;
  const int64_t block_stride = kBlockTokens * row_stride;
  const int blocks_per_seq = s.tokens / kBlockTokens;
  const int parts = s.tokens / s.part_tokens;
  const int job_blocks = s.part_tokens / kBlockTokens;
  const int64_t jobs = int64_t{s.seqs} * kHeads * parts;
  const int64_t blocks = int64_t{s.seqs} * blocks_per_seq;
  const int64_t cache_bytes = blocks * block_stride;  // one of K, V
  const int64_t region_bytes = 2 * cache_bytes;
  const int64_t regions = pool_bytes / region_bytes;
  if (s.tokens % s.part_tokens != 0 || s.part_tokens % kBlockTokens != 0 || job_blocks > kMaxJobBlocks ||
      job_blocks % U != 0 || job_blocks < U || regions < 1 || jobs * kThreads > sink_words ||
      (s.xcd && jobs % (8 * kHeads) != 0) || blocks > (int64_t{1} << 31) - 1) {
    std::fprintf(stderr, "paged: unsupported shape %s\n", s.name);
    std::exit(2);
  }
  // A shuffled assignment of the region's blocks to (sequence, block) slots.
  std::vector<int> table(static_cast<size_t>(blocks));
  std::iota(table.begin(), table.end(), 0);
  std::mt19937_64 rng(20261202);
  std::shuffle(table.begin(), table.end(), rng);
  int* d_table = nullptr;
  CHECK(hipMalloc(&d_table, table.size() * sizeof(int)));
  CHECK(hipMemcpy(d_table, table.data(), table.size() * sizeof(int), hipMemcpyHostToDevice));
  const double us = time_launches(
      [&](int i) {
        PagedArgs a;
        a.k = pool + (i % regions) * region_bytes;
        a.v = a.k + cache_bytes;
        a.table = d_table;
        a.seqs = s.seqs;
        a.heads = kHeads;
        a.blocks_per_seq = blocks_per_seq;
        a.part_tokens = s.part_tokens;
        a.parts = parts;
        a.row_stride = row_stride;
        a.block_stride = block_stride;
        a.xcd = s.xcd;
        paged_kernel<U><<<static_cast<unsigned>(jobs), kThreads>>>(a, sink);
      },
      iterations_for(region_bytes));
  CHECK(hipFree(d_table));
  std::printf("{\"pattern\": \"paged\", \"shape\": \"%s\", \"bytes\": %lld, \"workgroups\": %lld, "
              "\"partition_tokens\": %d, \"xcd_grouped\": %d, \"loads_in_flight\": %d, \"us\": %.2f, \"GBps\": %.0f}\n",
              s.name, static_cast<long long>(region_bytes), static_cast<long long>(jobs), s.part_tokens, s.xcd, U,
              us, region_bytes / (us * 1e3));
  std::fflush(stdout);
}

}  // namespace

int main() {
  // 5 GiB pool: the 4.3 GB paged shape fits once; small shapes rotate over >= 768 MB of regions.
  const int64_t pool_bytes = int64_t{5} << 30;
  const int64_t sink_words = int64_t{16384} * kThreads;
  unsigned char* pool = nullptr;
  uint32_t* sink = nullptr;
  CHECK(hipMalloc(&pool, pool_bytes));
  CHECK(hipMalloc(&sink, sink_words * sizeof(uint32_t)));
  CHECK(hipMemset(pool, 1, pool_bytes));
  CHECK(hipDeviceSynchronize());
  const int64_t small = int64_t{32} << 20;  // 33.5 MB: the 8-sequence, 1024-token decode's KV bytes
  // Small-pool views so that a small launch rotates over 1 GiB, not the whole pool (the rotation
  // already exceeds the last-level cache fourfold).
  const int64_t small_pool = int64_t{1} << 30;
  for (int groups : {64, 128, 256, 512, 1024, 2048}) {
    stream_case<4>(pool, small_pool, sink, sink_words, groups, small);
    if (small / groups / 16 / kThreads >= 8) stream_case<8>(pool, small_pool, sink, sink_words, groups, small);
    if (small / groups / 16 / kThreads >= 16) stream_case<16>(pool, small_pool, sink, sink_words, groups, small);
  }
  const int64_t large = int64_t{4} << 30;
  stream_case<8>(pool, pool_bytes, sink, sink_words, 8192, large);
  stream_case<16>(pool, pool_bytes, sink, sink_words, 8192, large);
  const PagedShape b8{"8 sequences x 1024 tokens, partitions of 256", 8, 1024, 256, 0};
  const PagedShape b8p128{"8 sequences x 1024 tokens, partitions of 128", 8, 1024, 128, 0};
  const PagedShape b128{"128 sequences x 8192 tokens, partitions of 2048", 128, 8192, 2048, 1};
  const PagedShape b128_flat{"128 sequences x 8192 tokens, partitions of 2048, identity placement", 128, 8192, 2048,
                             0};
  paged_case<2>(pool, small_pool, sink, sink_words, b8);
  paged_case<4>(pool, small_pool, sink, sink_words, b8);
  paged_case<8>(pool, small_pool, sink, sink_words, b8);
  paged_case<2>(pool, small_pool, sink, sink_words, b8p128);
  paged_case<4>(pool, small_pool, sink, sink_words, b8p128);
  paged_case<8>(pool, small_pool, sink, sink_words, b8p128);
  paged_case<4>(pool, pool_bytes, sink, sink_words, b128);
  paged_case<8>(pool, pool_bytes, sink, sink_words, b128);
  paged_case<16>(pool, pool_bytes, sink, sink_words, b128);
  paged_case<8>(pool, pool_bytes, sink, sink_words, b128_flat);
  CHECK(hipFree(pool));
  CHECK(hipFree(sink));
  return 0;
}
