// Declarations shared by the paged-attention decode host code (pa_decode_gfx950.hip) and its kernel
// units (pa_decode_kernels.hip, compiled once per element type and head_dim): launch limits, the
// kernel parameter block and the per-unit launch entry points.
#pragma once

#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdint.h>

namespace rk_pa {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kTile = 16;             // tokens per wave step = MFMA M
// Block-table entries of one partition's slice.  The host admits partition_tokens / block_size <=
// 512.  For block sizes up to 16 the partition size is a multiple of the block size, so a slice holds
// exactly partition_tokens / block_size entries; for larger blocks partition_tokens <= 8192 keeps it
// to 8192 / 32 + 1 = 257, the one extra entry being a block that straddles the partition start.
constexpr int kMaxSliceBlocks = 512;
// Partition growth stops at 256 blocks per partition.  Growth is balanced on sizes up to that many
// blocks; wider slices serve explicit partition sizes such as the 8192-token partitions of long
// 16-token-block contexts.
constexpr int kGrowMaxSliceBlocks = 256;
// Work-queue schedule limits: sequences and partition levels whose item map fits in LDS.
constexpr int kQueueMaxBatch = 1024;
constexpr int kQueueMaxLevels = 256;
// Larger batches run as launches of kQueueMaxBatch sequences; workspace header words 1 .. 63 hold the
// partition size each launch ran under partition growth.
constexpr int kQueueMaxLaunches = 63;
// Smallest partition the automatic choice runs on the queue.  Below it items are a tile or two per
// wave and the queue's per-item claim and barriers cost more than the grid's launches: 1024
// sequences of 64-512 tokens at P 64 measured 654 against 629 us, of 64-1024 tokens at P 128 709
// against 701 us; at P 256 every shape measured tied or won (1024 x 256-2048 tokens: 1061 against
// 1113 us).
constexpr int kQueueMinPartitionTokens = 256;
constexpr size_t kQueueHeaderBytes = 256;  // workspace bytes in front of the split-K records
// Partition growth (RK_PA_PARTITION_GROW): the queue kernel doubles the partition size P while
// P^2 <= kGrowBalance * W, W = context tokens x head slots per resident workgroup, up to
// kGrowMaxTokens.  Each item costs a fixed prologue and epilogue and the last items to finish set a
// tail of about one item, so the best size grows as sqrt(W).  Over eleven batches (16-1024 sequences
// of 1 to 64k tokens) the fastest of the fixed sizes 256-4096 bounds the constant to [1350, 1531);
// inside it the rule picks that size on all eleven.
constexpr int64_t kGrowBalance = 1440;
constexpr int kGrowMaxTokens = 4096;
constexpr int kGrowMaxSteps = 8;  // 16 << 8 = 4096
constexpr float kLog2e = 1.4426950408889634f;
// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector memory operations are
// outstanding: vmcnt in bits [3:0] and [15:14], expcnt [6:4] = 7 and lgkmcnt [11:8] = 15 (no wait on
// those counters).  Vector memory loads, LDS DMA included, retire in issue order, so vmcnt <= n
// means everything but the n most recently issued operations has landed.
constexpr int wait_vmcnt(int n) { return 0x0F70 | (n & 0xF) | ((n >> 4) << 14); }
// ... and the one that waits for lgkmcnt == 0 only (LDS and scalar memory), vmcnt left at its maximum.
constexpr int kWaitLgkmcnt0 = 0xC07F;

// ---------------------------------------------------------------------------------------------
// ---------------------------------------------------------------------------------------------
struct Params {
  const uint16_t* __restrict__ q;
  const uint16_t* __restrict__ k;
  const uint16_t* __restrict__ v;
  const void* __restrict__ block_tables;
  const void* __restrict__ context_lengths;
  uint16_t* __restrict__ out;
  float* __restrict__ ws_acc;  // [batch, query_heads, num_partitions, D]
  float* __restrict__ ws_ml;   // [batch, query_heads, num_partitions, 2] = (max, sum)
  // Fused merge only (else null): [batch, kv_heads * head_chunks] arrival counters, zero on entry,
  // left zero on exit (the last arriver resets its counter).
  uint32_t* __restrict__ counters;
  // Append-and-decode only (else null): [batch, kv_heads, D] K and V rows of each sequence's new
  // token (position context_length - 1).  The kernel attends to them from these buffers and stores
  // them into that position's cache slot; k_store / v_store are the caches' base addresses.
  const uint16_t* __restrict__ new_k;
  const uint16_t* __restrict__ new_v;
  uint16_t* k_store;
  uint16_t* v_store;
  int64_t block_stride;        // elements between physical blocks: BS * Hkv * D
  int64_t row_stride;          // elements between slots of a block: Hkv * D
  int32_t batch;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t group;        // query heads per KV head
  int32_t head_chunks;  // ceil(group / GC)
  int32_t num_blocks;
  int32_t max_blocks;
  int32_t bs_log2;
  int32_t partition_tokens;
  int32_t num_partitions;  // ceil(max_blocks * BS / partition_tokens)
  int32_t index_is64;
  float scale_log2e;
  // Work-queue schedule only (else null), last so the fields before them keep the grid kernel's
  // argument layout.  queue: the ticket counter.  queue_done: null when the counter sits in the
  // workspace header and pa_queue_reset_kernel zeroes it in front of every launch; otherwise (fused
  // launch: both words at the end of the arrival-counter array, zero on entry) the workgroups count
  // their exits on it and the last one zeroes both words for the next call.
  uint32_t* __restrict__ queue;
  uint32_t* __restrict__ queue_done;
  // Partition growth (work-queue schedule with RK_PA_PARTITION_GROW only; else null / 0): the queue
  // kernel runs partitions of partition_tokens << k tokens, at most grow_max_tokens, k chosen from
  // the context lengths.  grown: two-launch form only, workspace header word 1 + launch, where workgroup 0
  // stores the partition size it ran for the reduce kernel.
  uint32_t* __restrict__ grown;
  int32_t grow_max_tokens;
};

// Schedule requests (the RK_PA_SCHEDULE_* bits of the variant argument).
constexpr int kScheduleAuto = 0;
constexpr int kScheduleGrid = 1;
constexpr int kScheduleQueue = 2;

// How one call launches: its work items, schedule request, queue eligibility and stream; with
// `chosen`, only the partition kernel's schedule is decided (and stored there), nothing launched.
struct Launch {
  int64_t items;
  int schedule;
  bool queue_ok;
  hipStream_t stream;
  int* chosen;
};

// One launcher per (element type, head_dim), each defined in its own compilation of
// pa_decode_kernels.hip: the launches of one call (partition kernel and, when `reduce`, the merge
// kernel) for head chunk `gc` and kernel variant `variant`.  With `l.chosen`, nothing is launched:
// the partition kernel's schedule is stored there.
#define RK_PA_UNIT_LAUNCHER(ELEMENT, HEAD_DIM)                                                            \
  hipError_t launch_##ELEMENT##_d##HEAD_DIM(const Params& prm, int gc, int variant, const Launch& l, \
                                            bool partitions, bool reduce)
RK_PA_UNIT_LAUNCHER(bf16, 64);
RK_PA_UNIT_LAUNCHER(bf16, 128);
RK_PA_UNIT_LAUNCHER(bf16, 256);
RK_PA_UNIT_LAUNCHER(fp16, 64);
RK_PA_UNIT_LAUNCHER(fp16, 128);
RK_PA_UNIT_LAUNCHER(fp16, 256);

}  // namespace rk_pa
