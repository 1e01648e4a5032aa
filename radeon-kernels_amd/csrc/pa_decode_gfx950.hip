// Paged-attention decode for MI355X (gfx950): host side of the C ABI (include/rk_paged_attention.h).
//
// Validates shapes and pointers, lays out the split-K workspace, picks the head chunk, schedule and
// partition size, and launches the kernels of pa_decode_kernels.hip through the per-(element type,
// head_dim) launchers declared in pa_decode_common.hpp.  Also holds the allocation-free entry's
// device-resident scratch array.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "pa_decode_common.hpp"
#include "rk_paged_attention.h"

namespace {

using namespace rk_pa;

// ---------------------------------------------------------------------------------------------
// Host side.
thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buffer[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_last_error = buffer;
  return code;
}

// Query heads per workgroup: 8 for groups of 8 or more (each KV row is then read once per 8 query
// heads), else up to 4.  At head_dim 64 and 128 that held for every variant (1.3-1.75x faster than two
// chunks of 4).  At head_dim 256 it holds only with PV on MFMA, where a lane keeps 4 of the 8 heads'
// accumulators; with PV on fp32 FMAs the 8-head accumulators spill there, and those variants keep
// chunks of 4 (their 8-head head_dim 256 kernels are not built).
int head_chunk_for(int64_t group, int64_t head_dim, int variant) {
  if (group == 1) return 1;
  if (group == 2) return 2;
  return group >= 8 && (head_dim <= 128 || variant == RK_PA_VARIANT_MFMA) ? 8 : 4;
}

int log2_exact(int64_t x) {
  int r = 0;
  while ((int64_t{1} << r) < x) ++r;
  return ((int64_t{1} << r) == x) ? r : -1;
}

struct Shape {
  int64_t batch, query_heads, kv_heads, head_dim, num_blocks, block_size, max_blocks, partition;
  int64_t num_partitions;
};

int check_shape(const Shape& s) {
  if (s.batch <= 0 || s.query_heads <= 0 || s.kv_heads <= 0 || s.num_blocks <= 0 ||
      s.block_size <= 0 || s.max_blocks <= 0)
    return fail(RK_ERR_INVALID_ARGUMENT, "tensor dimensions must be positive");
  if (s.head_dim != 64 && s.head_dim != 128 && s.head_dim != 256)
    return fail(RK_ERR_INVALID_ARGUMENT, "head_dim must be one of 64, 128, 256 (got %lld)",
                static_cast<long long>(s.head_dim));
  if (s.query_heads % s.kv_heads != 0)
    return fail(RK_ERR_INVALID_ARGUMENT, "query_heads must be divisible by kv_heads");
  if (log2_exact(s.block_size) < 0 || s.block_size > 256)
    return fail(RK_ERR_UNSUPPORTED, "block_size must be a power of two <= 256 (got %lld)",
                static_cast<long long>(s.block_size));
  if (s.partition < kTile || s.partition > 8192 || s.partition % kTile != 0)
    return fail(RK_ERR_INVALID_ARGUMENT,
                "partition_tokens must be a multiple of 16 in [16, 8192] (got %lld)",
                static_cast<long long>(s.partition));
  if (s.partition / s.block_size > kMaxSliceBlocks)
    return fail(RK_ERR_INVALID_ARGUMENT, "partition_tokens / block_size must be <= %d", kMaxSliceBlocks);
  if (16 * s.kv_heads * s.head_dim >= (int64_t{1} << 30))
    return fail(RK_ERR_UNSUPPORTED, "kv_heads * head_dim is too large for this kernel");
  if (s.num_blocks >= (int64_t{1} << 31) || s.max_blocks * s.block_size >= (int64_t{1} << 31) ||
      s.batch >= (int64_t{1} << 31) || s.query_heads >= (int64_t{1} << 20))
    return fail(RK_ERR_UNSUPPORTED, "shape exceeds the 32-bit index range of this kernel");
  return RK_OK;
}

int64_t partitions_for(const Shape& s) {
  return (s.max_blocks * s.block_size + s.partition - 1) / s.partition;
}

// Workspace layout: a 256-byte header (word 0: the work-queue ticket counter; word 1 + i: the
// partition size launch i of a growing call ran, for the reduce kernel), partition
// accumulators (fp32, padded to 256 B), then partition (max, sum) pairs.
size_t acc_bytes_for(const Shape& s) {
  const size_t records = static_cast<size_t>(s.batch) * s.query_heads * s.num_partitions;
  return (records * s.head_dim * sizeof(float) + 255) & ~size_t{255};
}

size_t workspace_for(const Shape& s) {
  if (s.num_partitions <= 1) return 0;
  const size_t records = static_cast<size_t>(s.batch) * s.query_heads * s.num_partitions;
  return kQueueHeaderBytes + acc_bytes_for(s) + records * 2 * sizeof(float);
}

// QK^T on MFMA (PV on MFMA or on the vector ALUs): the variants the work queue, partition growth and
// append-and-decode are built for.
bool is_mfma(int variant) { return variant == RK_PA_VARIANT_MFMA || variant == RK_PA_VARIANT_MFMA_QK; }

// The work-queue schedule needs the workspace header (split-K shapes) and an item map that fits in
// the queue kernel's LDS; the VALU variant is not built for it.
bool queue_eligible(const Shape& s, int variant) {
  return is_mfma(variant) && s.num_partitions > 1 && s.num_partitions <= kQueueMaxLevels &&
         s.batch <= kQueueMaxBatch * kQueueMaxLaunches;
}

int queue_unsupported() {
  return fail(RK_ERR_UNSUPPORTED,
              "the work-queue schedule needs the MFMA variant, more than one partition per sequence "
              "(at most %d) and at most %d sequences", kQueueMaxLevels, kQueueMaxBatch * kQueueMaxLaunches);
}

// Counters of the fused launch: one 32-bit arrival counter per (sequence, KV head, chunk of up to 4
// query heads), then the work queue's ticket and exit counters.  The count does not depend on
// head_dim (rk_pa_decode_counter_words takes none): calls with 8-head chunks use a prefix of the
// arrival counters, and the queue words stay where this count puts them.
constexpr int64_t kQueueCounterWords = 2;
int64_t arrival_words_for(int64_t batch, int64_t query_heads, int64_t kv_heads) {
  const int64_t group = query_heads / kv_heads;
  const int64_t gc = group == 1 ? 1 : (group == 2 ? 2 : 4);  // 8-head chunks use fewer
  return batch * kv_heads * ((group + gc - 1) / gc);
}
int64_t counter_words_for(int64_t batch, int64_t query_heads, int64_t kv_heads) {
  return arrival_words_for(batch, query_heads, kv_heads) + kQueueCounterWords;
}

// The launcher of the unit compiled for this element type and head_dim.
hipError_t launch_unit(int dtype, int64_t head_dim, const Params& prm, int gc, int variant, const Launch& l,
                       bool partitions, bool reduce) {
  if (dtype == RK_DTYPE_BF16) {
    if (head_dim == 64) return launch_bf16_d64(prm, gc, variant, l, partitions, reduce);
    if (head_dim == 128) return launch_bf16_d128(prm, gc, variant, l, partitions, reduce);
    return launch_bf16_d256(prm, gc, variant, l, partitions, reduce);
  }
  if (head_dim == 64) return launch_fp16_d64(prm, gc, variant, l, partitions, reduce);
  if (head_dim == 128) return launch_fp16_d128(prm, gc, variant, l, partitions, reduce);
  return launch_fp16_d256(prm, gc, variant, l, partitions, reduce);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" int rk_pa_decode_workspace_bytes(int64_t batch, int64_t query_heads, int64_t head_dim,
                                            int64_t block_size, int64_t max_blocks_per_sequence,
                                            int64_t partition_tokens, size_t* bytes) {
  if (bytes == nullptr) return fail(RK_ERR_INVALID_ARGUMENT, "bytes must not be NULL");
  Shape s{batch, query_heads, 1, head_dim, 1, block_size, max_blocks_per_sequence, partition_tokens, 0};
  const int status = check_shape(s);
  if (status != RK_OK) return status;
  s.num_partitions = partitions_for(s);
  *bytes = workspace_for(s);
  return RK_OK;
}

extern "C" int rk_pa_decode_counter_words(int64_t batch, int64_t query_heads, int64_t kv_heads,
                                          size_t* words) {
  if (words == nullptr) return fail(RK_ERR_INVALID_ARGUMENT, "words must not be NULL");
  if (batch <= 0 || query_heads <= 0 || kv_heads <= 0)
    return fail(RK_ERR_INVALID_ARGUMENT, "tensor dimensions must be positive");
  if (query_heads % kv_heads != 0)
    return fail(RK_ERR_INVALID_ARGUMENT, "query_heads must be divisible by kv_heads");
  *words = static_cast<size_t>(counter_words_for(batch, query_heads, kv_heads));
  return RK_OK;
}

namespace {

// ---------------------------------------------------------------------------------------------
// Allocation-free decode: rk_pa_decode with its split-K records in a library-owned device array.
//
// `scratch` is a file-scope device array; every GPU the library runs on holds its own copy (at its
// own address) from the first call on that GPU until the process ends.  In host code the array's
// name is only a host-side stand-in, never a device address: the device address is looked up once
// per device with hipGetSymbolAddress, with that device current, and kept in g_scratch_ptr.  Only
// that pointer ever reaches a kernel.  The two-launch form needs nothing zeroed: the partition
// kernel writes every record the reduce kernel reads.
static __device__ __align__(256) unsigned char scratch[RK_PA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 256;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

// Device address of this device's `scratch`, looked up on the first call per device.
int scratch_address(void* stream, void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(RK_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (stream != nullptr) {
    int stream_device = -1;
    err = hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_device);
    if (err != hipSuccess)
      return fail(RK_ERR_INVALID_ARGUMENT, "hipStreamGetDevice failed: %s", hipGetErrorString(err));
    if (stream_device != device)
      return fail(RK_ERR_INVALID_ARGUMENT, "stream belongs to device %d but device %d is current",
                  stream_device, device);
  }
  if (device < 0 || device >= kMaxDevices)
    return fail(RK_ERR_UNSUPPORTED, "device index %d is outside [0, %d)", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail(RK_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                  hipGetErrorString(err));
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return RK_OK;
}

constexpr int kPhasePartitions = 1;
constexpr int kPhaseReduce = 2;
constexpr int kPhaseFused = 4;  // partition kernel merging in its last workgroups; no reduce launch
constexpr int kPhaseAppend = 8; // partition kernel also writes each sequence's new token (AP)
constexpr int kPhaseScratch = 16; // records in this device's `scratch` array, not `workspace`

// The variant argument's kernel variant (low byte) and RK_PA_SCHEDULE_* request.
int split_variant(int* variant, int* schedule, bool* grow = nullptr) {
  const int bits = *variant;
  if ((bits & ~(RK_PA_SCHEDULE_GRID | RK_PA_SCHEDULE_QUEUE | RK_PA_PARTITION_GROW | 0xFF)) != 0 ||
      (bits & (RK_PA_SCHEDULE_GRID | RK_PA_SCHEDULE_QUEUE)) == (RK_PA_SCHEDULE_GRID | RK_PA_SCHEDULE_QUEUE) ||
      (!is_mfma(bits & 0xFF) && (bits & 0xFF) != RK_PA_VARIANT_VALU))
    return fail(RK_ERR_INVALID_ARGUMENT, "unknown kernel variant %d", bits);
  *schedule = (bits & RK_PA_SCHEDULE_QUEUE) != 0 ? kScheduleQueue
              : (bits & RK_PA_SCHEDULE_GRID) != 0 ? kScheduleGrid
                                                  : kScheduleAuto;
  if (grow != nullptr) *grow = (bits & RK_PA_PARTITION_GROW) != 0;
  *variant = bits & 0xFF;
  return RK_OK;
}

// Partition growth's smallest size for a table too wide for the queue's item map at partition_tokens
// (more than kQueueMaxLevels partitions): the first doubling that fits, within kGrowMaxTokens and 256
// blocks.  The call then runs, and lays out its records, as if given that size; a call the queue
// cannot take anyway (grid schedule requested, VALU variant, too many sequences) is left unchanged.
void grow_base(Shape* s, int variant, int schedule, bool grow) {
  if (!grow || schedule == kScheduleGrid || !is_mfma(variant) ||
      s->batch > int64_t{kQueueMaxBatch} * kQueueMaxLaunches ||
      s->num_partitions <= kQueueMaxLevels)
    return;
  const int64_t table_tokens = s->max_blocks * s->block_size;
  int64_t base = s->partition;
  while ((table_tokens + base - 1) / base > kQueueMaxLevels) {
    base *= 2;
    if (base > kGrowMaxTokens || base / s->block_size > kGrowMaxSliceBlocks) return;
  }
  s->partition = base;
  s->num_partitions = partitions_for(*s);
}

// Largest partition size partition growth may reach: partition_tokens doubled while it stays within
// kGrowMaxTokens and 256 blocks and leaves the table at least two partitions; 0 when no doubling
// fits.
int32_t grow_limit(const Shape& s) {
  const int64_t table_tokens = s.max_blocks * s.block_size;
  int64_t limit = s.partition;
  for (int k = 0; k < kGrowMaxSteps; ++k) {
    const int64_t next = limit * 2;
    if (next > kGrowMaxTokens || next / s.block_size > kGrowMaxSliceBlocks || next >= table_tokens) break;
    limit = next;
  }
  return limit > s.partition ? static_cast<int32_t>(limit) : 0;
}

int decode_phases(const void* query, const void* key_cache, const void* value_cache,
                  const void* block_tables, const void* context_lengths, void* output, void* workspace,
                  size_t workspace_bytes, int64_t batch, int64_t query_heads, int64_t kv_heads,
                  int64_t head_dim, int64_t num_blocks, int64_t block_size,
                  int64_t max_blocks_per_sequence, float scale, int dtype, int index_dtype,
                  int64_t partition_tokens, int variant, void* stream, int phases,
                  uint32_t* counters = nullptr, size_t counter_words = 0,
                  const void* new_key = nullptr, const void* new_value = nullptr) {
  if (!query || !key_cache || !value_cache || !block_tables || !context_lengths || !output)
    return fail(RK_ERR_INVALID_ARGUMENT, "tensor pointers must not be NULL");
  const bool append = (phases & kPhaseAppend) != 0;
  if (append && (!new_key || !new_value))
    return fail(RK_ERR_INVALID_ARGUMENT, "new_key and new_value must not be NULL");
  if (append && !is_mfma(variant & 0xFF))
    return fail(RK_ERR_UNSUPPORTED, "append-and-decode is built for RK_PA_VARIANT_MFMA and RK_PA_VARIANT_MFMA_QK only");
  if (append && (!aligned16(new_key) || !aligned16(new_value)))
    return fail(RK_ERR_UNSUPPORTED, "new_key and new_value must be 16-byte aligned");
  if (dtype != RK_DTYPE_FP16 && dtype != RK_DTYPE_BF16)
    return fail(RK_ERR_INVALID_ARGUMENT, "dtype must be RK_DTYPE_FP16 or RK_DTYPE_BF16");
  if (index_dtype != RK_INDEX_INT32 && index_dtype != RK_INDEX_INT64)
    return fail(RK_ERR_INVALID_ARGUMENT, "index_dtype must be RK_INDEX_INT32 or RK_INDEX_INT64");
  int schedule = kScheduleAuto;
  bool grow = false;
  if (split_variant(&variant, &schedule, &grow) != RK_OK) return RK_ERR_INVALID_ARGUMENT;
  if (!(scale > 0.0f) || !isfinite(scale))
    return fail(RK_ERR_INVALID_ARGUMENT, "scale must be positive and finite");
  if (!aligned16(query) || !aligned16(key_cache) || !aligned16(value_cache) || !aligned16(output))
    return fail(RK_ERR_UNSUPPORTED, "query, caches and output must be 16-byte aligned");

  Shape s{batch, query_heads, kv_heads, head_dim, num_blocks, block_size, max_blocks_per_sequence,
          partition_tokens, 0};
  int status = check_shape(s);
  if (status != RK_OK) return status;
  s.num_partitions = partitions_for(s);
  grow_base(&s, variant, schedule, grow);
  partition_tokens = s.partition;
  const size_t need = workspace_for(s);
  if ((phases & kPhaseScratch) != 0) {
    if (need > RK_PA_NOALLOC_SCRATCH_BYTES)
      return fail(RK_ERR_WORKSPACE,
                  "this shape needs %zu bytes of split-K scratch; rk_pa_decode_noalloc holds %zu "
                  "(use a larger partition_tokens, or rk_pa_decode with a workspace)",
                  need, static_cast<size_t>(RK_PA_NOALLOC_SCRATCH_BYTES));
    workspace = nullptr;
    workspace_bytes = 0;
    if (need > 0) {
      status = scratch_address(stream, &workspace);
      if (status != RK_OK) return status;
      workspace_bytes = RK_PA_NOALLOC_SCRATCH_BYTES;
    }
  }
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(RK_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                workspace_bytes);
  if (need > 0 && (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(RK_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  // The fused launch needs its counters only when some sequence can span several partitions.
  const bool fused = (phases & kPhaseFused) != 0 && need > 0;
  if (fused) {
    const size_t words = static_cast<size_t>(counter_words_for(batch, query_heads, kv_heads));
    if (counters == nullptr || counter_words < words)
      return fail(RK_ERR_WORKSPACE, "%zu counter words required, %zu given", words, counter_words);
    if ((reinterpret_cast<uintptr_t>(counters) & 3u) != 0)
      return fail(RK_ERR_WORKSPACE, "counters must be 4-byte aligned");
  }

  const int64_t group = query_heads / kv_heads;
  const int gc = head_chunk_for(group, head_dim, variant);
  const int64_t head_chunks = (group + gc - 1) / gc;
  const int64_t grid = batch * kv_heads * head_chunks * s.num_partitions;  // one workgroup per work item
  if (grid >= (int64_t{1} << 31))
    return fail(RK_ERR_UNSUPPORTED, "launch grid exceeds 2^31 workgroups");

  Params prm{};
  prm.q = static_cast<const uint16_t*>(query);
  prm.k = static_cast<const uint16_t*>(key_cache);
  prm.v = static_cast<const uint16_t*>(value_cache);
  prm.block_tables = block_tables;
  prm.context_lengths = context_lengths;
  prm.out = static_cast<uint16_t*>(output);
  if (need > 0) {
    char* records = static_cast<char*>(workspace) + kQueueHeaderBytes;
    prm.ws_acc = reinterpret_cast<float*>(records);
    prm.ws_ml = reinterpret_cast<float*>(records + acc_bytes_for(s));
  }
  const bool partitions = (phases & (kPhasePartitions | kPhaseFused)) != 0;
  // A batch larger than the queue's item map runs as launches of kQueueMaxBatch sequences (the last
  // one shorter), in stream order on offset views of the same buffers.  Each picks its own schedule
  // (and grown size), so every launch is a queue-eligible shape.
  const int64_t rows_per_launch =
      batch > kQueueMaxBatch && schedule != kScheduleGrid && queue_eligible(s, variant) ? kQueueMaxBatch : batch;
  Shape first = s;
  first.batch = rows_per_launch;
  const bool queue = partitions && schedule != kScheduleGrid && queue_eligible(first, variant);
  if (partitions && schedule == kScheduleQueue && !queue) return queue_unsupported();
  if (queue && fused) {  // the ticket and exit counters after the arrival counters, zero on entry
    prm.queue = counters + arrival_words_for(batch, query_heads, kv_heads);
    prm.queue_done = prm.queue + 1;
  } else if (queue) {  // the workspace header, zeroed by a kernel in front of the launch
    prm.queue = static_cast<uint32_t*>(workspace);
  }
  prm.counters = fused ? counters : nullptr;
  if (append) {
    prm.new_k = static_cast<const uint16_t*>(new_key);
    prm.new_v = static_cast<const uint16_t*>(new_value);
    prm.k_store = static_cast<uint16_t*>(const_cast<void*>(key_cache));
    prm.v_store = static_cast<uint16_t*>(const_cast<void*>(value_cache));
  }
  prm.block_stride = block_size * kv_heads * head_dim;
  prm.row_stride = kv_heads * head_dim;
  prm.query_heads = static_cast<int32_t>(query_heads);
  prm.kv_heads = static_cast<int32_t>(kv_heads);
  prm.group = static_cast<int32_t>(group);
  prm.head_chunks = static_cast<int32_t>(head_chunks);
  prm.num_blocks = static_cast<int32_t>(num_blocks);
  prm.max_blocks = static_cast<int32_t>(max_blocks_per_sequence);
  prm.bs_log2 = log2_exact(block_size);
  prm.partition_tokens = static_cast<int32_t>(partition_tokens);
  prm.num_partitions = static_cast<int32_t>(s.num_partitions);
  prm.index_is64 = index_dtype == RK_INDEX_INT64 ? 1 : 0;
  prm.scale_log2e = scale * kLog2e;

  const bool reduce = !fused && (phases & kPhaseReduce) != 0 && s.num_partitions > 1;
  const int64_t index_bytes = index_dtype == RK_INDEX_INT64 ? 8 : 4;
  const int64_t heads_per_seq = kv_heads * head_chunks;
  for (int64_t launch = 0, b0 = 0; b0 < batch; ++launch, b0 += rows_per_launch) {
    const int64_t rows = std::min(rows_per_launch, batch - b0);
    Params cp = prm;
    cp.batch = static_cast<int32_t>(rows);
    cp.q = prm.q + b0 * query_heads * head_dim;
    cp.out = prm.out + b0 * query_heads * head_dim;
    cp.block_tables = static_cast<const char*>(block_tables) + b0 * max_blocks_per_sequence * index_bytes;
    cp.context_lengths = static_cast<const char*>(context_lengths) + b0 * index_bytes;
    if (need > 0) {
      cp.ws_acc = prm.ws_acc + b0 * query_heads * s.num_partitions * head_dim;
      cp.ws_ml = prm.ws_ml + b0 * query_heads * s.num_partitions * 2;
    }
    if (fused) cp.counters = counters + b0 * heads_per_seq;
    if (append) {
      cp.new_k = prm.new_k + b0 * kv_heads * head_dim;
      cp.new_v = prm.new_v + b0 * kv_heads * head_dim;
    }
    const int64_t items = rows * heads_per_seq * s.num_partitions;
    Shape sc = s;
    sc.batch = rows;

    // Partition growth runs on the work-queue schedule only.  The dry run makes the partition
    // launch's own choice, also in a reduce-only call, which must read the size that launch ran
    // (header word 1 + launch).
    if (grow && schedule != kScheduleGrid && queue_eligible(sc, variant)) {
      const int32_t limit = grow_limit(sc);
      if (limit > 0) {
        int chosen = RK_PA_SCHEDULE_GRID;
        const Launch dry{items, schedule, true, nullptr, &chosen};
        const hipError_t err = launch_unit(dtype, head_dim, cp, gc, variant, dry, true, false);
        if (err != hipSuccess)
          return fail(RK_ERR_LAUNCH, "paged attention schedule query failed: %s", hipGetErrorString(err));
        if (chosen == RK_PA_SCHEDULE_QUEUE) {
          cp.grow_max_tokens = limit;
          if (!fused) cp.grown = static_cast<uint32_t*>(workspace) + 1 + launch;
        }
      }
    }

    const Launch l{items, schedule, queue, static_cast<hipStream_t>(stream), nullptr};
    const hipError_t err = launch_unit(dtype, head_dim, cp, gc, variant, l, partitions, reduce);
    if (err != hipSuccess)
      return fail(RK_ERR_LAUNCH, "paged attention launch failed: %s", hipGetErrorString(err));
  }
  return RK_OK;
}

}  // namespace

extern "C" int rk_pa_decode(const void* query, const void* key_cache, const void* value_cache,
                            const void* block_tables, const void* context_lengths, void* output,
                            void* workspace, size_t workspace_bytes, int64_t batch,
                            int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                            int64_t num_blocks, int64_t block_size,
                            int64_t max_blocks_per_sequence, float scale, int dtype,
                            int index_dtype, int64_t partition_tokens, int variant, void* stream) {
  return decode_phases(query, key_cache, value_cache, block_tables, context_lengths, output,
                       workspace, workspace_bytes, batch, query_heads, kv_heads, head_dim,
                       num_blocks, block_size, max_blocks_per_sequence, scale, dtype, index_dtype,
                       partition_tokens, variant, stream, kPhasePartitions | kPhaseReduce);
}

extern "C" int rk_pa_decode_partitions(const void* query, const void* key_cache,
                                       const void* value_cache, const void* block_tables,
                                       const void* context_lengths, void* output, void* workspace,
                                       size_t workspace_bytes, int64_t batch, int64_t query_heads,
                                       int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                                       int64_t block_size, int64_t max_blocks_per_sequence,
                                       float scale, int dtype, int index_dtype,
                                       int64_t partition_tokens, int variant, void* stream) {
  return decode_phases(query, key_cache, value_cache, block_tables, context_lengths, output,
                       workspace, workspace_bytes, batch, query_heads, kv_heads, head_dim,
                       num_blocks, block_size, max_blocks_per_sequence, scale, dtype, index_dtype,
                       partition_tokens, variant, stream, kPhasePartitions);
}

extern "C" int rk_pa_decode_reduce(const void* query, const void* key_cache,
                                   const void* value_cache, const void* block_tables,
                                   const void* context_lengths, void* output, void* workspace,
                                   size_t workspace_bytes, int64_t batch, int64_t query_heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                                   int64_t block_size, int64_t max_blocks_per_sequence,
                                   float scale, int dtype, int index_dtype,
                                   int64_t partition_tokens, int variant, void* stream) {
  return decode_phases(query, key_cache, value_cache, block_tables, context_lengths, output,
                       workspace, workspace_bytes, batch, query_heads, kv_heads, head_dim,
                       num_blocks, block_size, max_blocks_per_sequence, scale, dtype, index_dtype,
                       partition_tokens, variant, stream, kPhaseReduce);
}

extern "C" int rk_pa_decode_fused(const void* query, const void* key_cache, const void* value_cache,
                                  const void* block_tables, const void* context_lengths, void* output,
                                  void* workspace, size_t workspace_bytes, uint32_t* counters,
                                  size_t counter_words, int64_t batch, int64_t query_heads,
                                  int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                                  int64_t block_size, int64_t max_blocks_per_sequence, float scale,
                                  int dtype, int index_dtype, int64_t partition_tokens, int variant,
                                  void* stream) {
  return decode_phases(query, key_cache, value_cache, block_tables, context_lengths, output,
                       workspace, workspace_bytes, batch, query_heads, kv_heads, head_dim,
                       num_blocks, block_size, max_blocks_per_sequence, scale, dtype, index_dtype,
                       partition_tokens, variant, stream, kPhaseFused, counters, counter_words);
}

extern "C" int rk_pa_decode_append(const void* query, const void* new_key, const void* new_value,
                                   void* key_cache, void* value_cache, const void* block_tables,
                                   const void* context_lengths, void* output, void* workspace,
                                   size_t workspace_bytes, uint32_t* counters, size_t counter_words,
                                   int64_t batch, int64_t query_heads, int64_t kv_heads,
                                   int64_t head_dim, int64_t num_blocks, int64_t block_size,
                                   int64_t max_blocks_per_sequence, float scale, int dtype,
                                   int index_dtype, int64_t partition_tokens, int variant,
                                   void* stream) {
  const int phases = kPhaseAppend | (counters != nullptr ? kPhaseFused : kPhasePartitions | kPhaseReduce);
  return decode_phases(query, key_cache, value_cache, block_tables, context_lengths, output,
                       workspace, workspace_bytes, batch, query_heads, kv_heads, head_dim,
                       num_blocks, block_size, max_blocks_per_sequence, scale, dtype, index_dtype,
                       partition_tokens, variant, stream, phases, counters, counter_words, new_key,
                       new_value);
}

extern "C" int rk_pa_decode_noalloc(const void* query, const void* key_cache, const void* value_cache,
                                    const void* block_tables, const void* context_lengths, void* output,
                                    int64_t batch, int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                                    int64_t num_blocks, int64_t block_size,
                                    int64_t max_blocks_per_sequence, float scale, int dtype,
                                    int index_dtype, int64_t partition_tokens, int variant,
                                    void* stream) {
  return decode_phases(query, key_cache, value_cache, block_tables, context_lengths, output, nullptr, 0,
                       batch, query_heads, kv_heads, head_dim, num_blocks, block_size,
                       max_blocks_per_sequence, scale, dtype, index_dtype, partition_tokens, variant,
                       stream, kPhasePartitions | kPhaseReduce | kPhaseScratch);
}

extern "C" int rk_pa_decode_schedule(int64_t batch, int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                                     int64_t block_size, int64_t max_blocks_per_sequence, int dtype,
                                     int64_t partition_tokens, int variant, int* schedule) {
  if (schedule == nullptr) return fail(RK_ERR_INVALID_ARGUMENT, "schedule must not be NULL");
  if (dtype != RK_DTYPE_FP16 && dtype != RK_DTYPE_BF16)
    return fail(RK_ERR_INVALID_ARGUMENT, "dtype must be RK_DTYPE_FP16 or RK_DTYPE_BF16");
  int requested = kScheduleAuto;
  bool grow = false;
  if (split_variant(&variant, &requested, &grow) != RK_OK) return RK_ERR_INVALID_ARGUMENT;
  Shape s{batch, query_heads, kv_heads, head_dim, 1, block_size, max_blocks_per_sequence, partition_tokens, 0};
  const int status = check_shape(s);
  if (status != RK_OK) return status;
  s.num_partitions = partitions_for(s);
  grow_base(&s, variant, requested, grow);
  partition_tokens = s.partition;
  const bool queue = requested != kScheduleGrid && queue_eligible(s, variant);
  if (requested == kScheduleQueue && !queue) return queue_unsupported();
  const int64_t group = query_heads / kv_heads;
  const int gc = head_chunk_for(group, head_dim, variant);
  const int64_t rows = queue && batch > kQueueMaxBatch ? kQueueMaxBatch : batch;  // the first launch
  const int64_t items = rows * kv_heads * ((group + gc - 1) / gc) * s.num_partitions;
  Params prm{};
  prm.bs_log2 = log2_exact(block_size);
  prm.partition_tokens = static_cast<int32_t>(partition_tokens);
  int chosen = RK_PA_SCHEDULE_GRID;
  const Launch l{items, requested, queue, nullptr, &chosen};
  const hipError_t err = launch_unit(dtype, head_dim, prm, gc, variant, l, true, false);
  if (err != hipSuccess) return fail(RK_ERR_LAUNCH, "schedule query failed: %s", hipGetErrorString(err));
  *schedule = chosen;
  return RK_OK;
}

extern "C" const char* rk_pa_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* rk_pa_version(void) { return "rk_pa_gfx950 1.0.0 (gfx950, wave64)"; }
