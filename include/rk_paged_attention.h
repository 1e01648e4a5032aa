/*
 * rk_paged_attention.h -- C ABI of the gfx950 (MI355X) paged-attention decode library.
 *
 * Library: librk_pa_gfx950.so (hand-written HIP for CDNA4, wave64).  No torch types cross
 * this boundary: every tensor is a device pointer to a dense, contiguous buffer and every
 * size is an int64_t.  All calls are asynchronous on the given HIP stream and never read
 * device memory from the host, so they can be captured into a HIP graph.
 *
 * Reference interface each entry point replaces (zihaomu/radeon-kernels):
 *   rk_pa_decode            -> benchmarks/paged_attention/native_paged_attention.hip:191-242
 *                              (paged_attention_impl<W>, bound as attention_wave{1,4,8} at :244-283),
 *                              reached from src/radeon_kernels/providers/native.py:25 with the
 *                              arguments built at src/radeon_kernels/ops/paged_attention/api.py:117-124.
 *   rk_pa_decode_workspace_bytes
 *                           -> no reference counterpart: the reference kernel has no context split.
 *                              The caller sizes the split-K partial buffer with it (the torch
 *                              extension allocates it from the caching allocator).
 *   rk_pa_decode_fused, rk_pa_decode_counter_words
 *                           -> no reference counterpart: the single-launch form of rk_pa_decode for
 *                              callers that keep a small persistent counter buffer per stream
 *                              (the torch extension does).
 *   rk_pa_decode_append    -> no reference counterpart: kv_cache_append of each sequence's new token
 *                              (benchmarks/kv_cache/native_kv_cache.hip:22-51, one token per
 *                              sequence at position context_length - 1) followed by rk_pa_decode, in
 *                              the decode's own launch.
 *   rk_pa_decode_schedule  -> no reference counterpart: which partition-kernel schedule a call runs.
 *   rk_pa_last_error, rk_pa_version
 *                           -> error text that TORCH_CHECK carried in the reference
 *                              (native_paged_attention.hip:199-219,239-240).
 *
 * Tensor layouts (row-major, contiguous) -- identical to the reference contract
 * (contracts/paged_attention_decode-1.0.json:5-14):
 *   query           [batch, query_heads, head_dim]                      fp16 | bf16
 *   key_cache       [num_blocks, block_size, kv_heads, head_dim]        fp16 | bf16
 *   value_cache     [num_blocks, block_size, kv_heads, head_dim]        fp16 | bf16
 *   block_tables    [batch, max_blocks_per_sequence]                    int32 | int64
 *   context_lengths [batch]                                             int32 | int64
 *   output          [batch, query_heads, head_dim]                      dtype of query
 *
 * Semantics (src/radeon_kernels/ops/paged_attention/reference.py:7-47): query head h reads KV head
 * h / (query_heads / kv_heads); token t of sequence b lives in slot
 * block_tables[b, t / block_size] * block_size + t % block_size; tokens t >= context_length are
 * masked; softmax and both contractions accumulate in fp32; the result is rounded to the query
 * dtype.  context_length is clamped to max_blocks_per_sequence * block_size; a context length
 * <= 0 yields NaN (softmax over an empty set); tokens whose physical block id is outside
 * [0, num_blocks) are skipped and never dereferenced.
 */
#ifndef RK_PAGED_ATTENTION_H
#define RK_PAGED_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by every entry point. */
#define RK_OK 0
#define RK_ERR_INVALID_ARGUMENT 1 /* shapes, pointers or scalars violate the contract */
#define RK_ERR_UNSUPPORTED 2      /* valid for the operator but not for this kernel */
#define RK_ERR_WORKSPACE 3        /* workspace missing or smaller than required */
#define RK_ERR_LAUNCH 4           /* the HIP runtime rejected a launch */

/* Element types. */
#define RK_DTYPE_FP16 0
#define RK_DTYPE_BF16 1
#define RK_INDEX_INT32 0
#define RK_INDEX_INT64 1

/* Kernel variants: where QK^T and PV are computed.  All three give results within the operator's
 * tolerances.  PV on MFMA takes each fp32 probability as a rounded high part plus its residual
 * (about 2^-16 relative), so its products match the fp32 FMAs' to within fp32 accumulation. */
#define RK_PA_VARIANT_MFMA 0    /* QK^T and PV on v_mfma_f32_16x16x32_{bf16,f16} */
#define RK_PA_VARIANT_VALU 1    /* QK^T on fp32 FMAs + DPP row reductions, PV on fp32 FMAs */
#define RK_PA_VARIANT_MFMA_QK 2 /* QK^T on MFMA, PV on fp32 FMAs */

/*
 * Schedule of the partition kernel, OR-ed into the variant argument (no reference counterpart).
 * Without either bit the library chooses: the work queue when the call is eligible for it, its
 * work items (sequence x KV head x head chunk x partition) exceed the workgroups the device holds
 * at once and partition_tokens >= 256, else one workgroup per work item.  Both schedules compute every item the same way, so
 * outputs are bit-identical.
 *   RK_PA_SCHEDULE_GRID   one workgroup per work item, items past a sequence's context included
 *                         (they exit at once).
 *   RK_PA_SCHEDULE_QUEUE  as many workgroups as the device holds at once take the items that
 *                         hold tokens from a ticket counter: in the workspace header, zeroed by a
 *                         one-thread kernel launched first, or, for rk_pa_decode_fused and the fused
 *                         rk_pa_decode_append, in the last two words of the counter array, which the
 *                         launch's last workgroup leaves zero (one launch).  Eligible: RK_PA_VARIANT_MFMA or _MFMA_QK, a split-K shape
 *                         (rk_pa_decode_workspace_bytes > 0) with at most 256 partitions per
 *                         sequence and at most 64512 sequences; RK_ERR_UNSUPPORTED otherwise.
 * A batch of more than 1024 sequences on an eligible call runs as consecutive launches of 1024
 * sequences (the last shorter) on the same stream, each choosing its own schedule.
 */
#define RK_PA_SCHEDULE_GRID 0x100
#define RK_PA_SCHEDULE_QUEUE 0x200

/*
 * Partition growth, OR-ed into the variant argument (no reference counterpart): partition_tokens
 * becomes the smallest partition size.  When the work-queue schedule runs, its workgroups read the
 * context lengths and run partitions of P = partition_tokens * 2^k tokens, the largest k with
 * P^2 <= 1440 * W (W: the context tokens of all sequences, each clamped to the table, times the
 * head slots per sequence -- KV heads x head chunks -- divided by the workgroups of the launch),
 * within 4096 tokens, 256 blocks and fewer tokens than the table holds
 * (max_blocks_per_sequence * block_size).  A table wider than 256 partitions of partition_tokens
 * (too wide for the work queue) starts from the first doubling of partition_tokens that fits, if
 * one does within those limits, so long tables also run on the work queue.  Without the work queue
 * the bit changes nothing.  Records keep the layout of that smallest size, so the workspace
 * rk_pa_decode_workspace_bytes gives for partition_tokens suffices.  The two-launch forms keep the
 * size the partition launch ran in workspace header word 1 (word 1 + i for launch i of a batch of
 * more than 1024 sequences) for the reduce launch, so rk_pa_decode_partitions and
 * rk_pa_decode_reduce take the same variant.
 * The output is bit-identical to a call without the bit at partition_tokens * 2^k.
 */
#define RK_PA_PARTITION_GROW 0x400

/*
 * The schedule (RK_PA_SCHEDULE_GRID or RK_PA_SCHEDULE_QUEUE) that rk_pa_decode, its phase entries,
 * rk_pa_decode_fused and rk_pa_decode_noalloc run for these arguments on the current device (no
 * reference counterpart; for a batch run as launches of 1024 sequences, the first launch's).  The index dtype does not enter the choice.  Launches nothing; the first
 * query of a kernel configuration reads its occupancy from the runtime.
 */
int rk_pa_decode_schedule(int64_t batch, int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                          int64_t block_size, int64_t max_blocks_per_sequence, int dtype,
                          int64_t partition_tokens, int variant, int* schedule);

/*
 * Bytes of device workspace rk_pa_decode needs for this shape and partition size: a 256-byte
 * header (word 0: the work-queue ticket counter; words 1-63: the partition size each launch of a
 * growing call ran) and
 * the split-K partial (max, sum, accumulator) records,
 * fp32.  Zero when one partition covers max_blocks_per_sequence * block_size tokens (the
 * single-pass launch needs none).
 */
int rk_pa_decode_workspace_bytes(int64_t batch, int64_t query_heads, int64_t head_dim,
                                 int64_t block_size, int64_t max_blocks_per_sequence,
                                 int64_t partition_tokens, size_t* bytes);

/*
 * Paged-attention decode: one query token per sequence against the paged K/V cache.
 *
 * partition_tokens: context tokens per workgroup (split-K partition); a multiple of 16 in
 *   [16, 8192] with partition_tokens / block_size <= 512.
 * variant: RK_PA_VARIANT_MFMA, RK_PA_VARIANT_VALU or RK_PA_VARIANT_MFMA_QK, optionally OR-ed with one RK_PA_SCHEDULE_* bit
 *   and with RK_PA_PARTITION_GROW.
 * workspace/workspace_bytes: device buffer of at least rk_pa_decode_workspace_bytes(...) bytes
 *   (may be NULL/0 when that is zero).  Its contents need no initialisation.
 * stream: hipStream_t to launch on (NULL = the null stream).
 *
 * Supported by this library: head_dim in {64, 128, 256}; block_size a power of two in
 * [1, 256]; query_heads % kv_heads == 0; num_blocks < 2^31.
 */
int rk_pa_decode(const void* query, const void* key_cache, const void* value_cache,
                 const void* block_tables, const void* context_lengths, void* output,
                 void* workspace, size_t workspace_bytes, int64_t batch, int64_t query_heads,
                 int64_t kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                 int64_t max_blocks_per_sequence, float scale, int dtype, int index_dtype,
                 int64_t partition_tokens, int variant, void* stream);

/*
 * The two launches rk_pa_decode makes, callable separately with the same arguments (no reference
 * counterpart; the reference kernel is a single pass).  rk_pa_decode_partitions runs the split-K
 * partition kernel: it writes the final output of every sequence that fits in one partition and a
 * partial record of every other partition into the workspace.  rk_pa_decode_reduce then merges
 * those records into the output (it launches nothing when one partition covers
 * max_blocks_per_sequence * block_size).  Issued in that order on one stream they are exactly
 * rk_pa_decode; splitting them lets a caller time or schedule the phases individually.
 */
int rk_pa_decode_partitions(const void* query, const void* key_cache, const void* value_cache,
                            const void* block_tables, const void* context_lengths, void* output,
                            void* workspace, size_t workspace_bytes, int64_t batch,
                            int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                            int64_t num_blocks, int64_t block_size,
                            int64_t max_blocks_per_sequence, float scale, int dtype,
                            int index_dtype, int64_t partition_tokens, int variant, void* stream);
int rk_pa_decode_reduce(const void* query, const void* key_cache, const void* value_cache,
                        const void* block_tables, const void* context_lengths, void* output,
                        void* workspace, size_t workspace_bytes, int64_t batch,
                        int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                        int64_t num_blocks, int64_t block_size, int64_t max_blocks_per_sequence,
                        float scale, int dtype, int index_dtype, int64_t partition_tokens,
                        int variant, void* stream);

/*
 * Single-launch decode (no reference counterpart): the partition kernel merges the partition
 * records itself.  The last workgroup to finish a (sequence, KV head, head chunk) counts its arrival
 * on a device-scope atomic counter, sees that it was last, and merges the records of every
 * partition of that sequence in partition order; no reduce launch follows.  Results agree with
 * rk_pa_decode to fp32 rounding of the final merge (both are deterministic).
 *
 * counters/counter_words: device array of at least rk_pa_decode_counter_words(...) uint32 words: one
 *   arrival counter per (sequence, KV head, head chunk), then the work-queue schedule's ticket and exit
 *   counters.  It must be all zero before the first call (e.g. hipMemset once at allocation); every call
 *   that completes leaves it all zero again, so one buffer serves any number of calls in stream
 *   order.  Calls that may run concurrently (different streams) need separate counter buffers
 *   and separate workspaces.  Ignored (may be NULL) when rk_pa_decode_workspace_bytes is zero.
 * All other arguments are those of rk_pa_decode.
 */
int rk_pa_decode_counter_words(int64_t batch, int64_t query_heads, int64_t kv_heads, size_t* words);
int rk_pa_decode_fused(const void* query, const void* key_cache, const void* value_cache,
                       const void* block_tables, const void* context_lengths, void* output,
                       void* workspace, size_t workspace_bytes, uint32_t* counters,
                       size_t counter_words, int64_t batch, int64_t query_heads, int64_t kv_heads,
                       int64_t head_dim, int64_t num_blocks, int64_t block_size,
                       int64_t max_blocks_per_sequence, float scale, int dtype, int index_dtype,
                       int64_t partition_tokens, int variant, void* stream);

/*
 * Append-and-decode (no reference counterpart): one decode step of a serving loop in the decode's
 * launch.  Each sequence b has one new token at position context_lengths[b] - 1 (context lengths
 * already count it), i.e. in slot block_tables[b, t / block_size] * block_size + t % block_size.
 * The call stores new_key[b] / new_value[b] ([batch, kv_heads, head_dim], the dtype of the caches)
 * into that slot of key_cache / value_cache, exactly as kv_cache_append with that slot mapping
 * would, and attends over the context with the new token read from new_key / new_value: outputs
 * and caches are bit-identical to the append followed by rk_pa_decode (or rk_pa_decode_fused).
 *
 * Preconditions beyond rk_pa_decode's: no other sequence of the call attends to a new token's slot
 * (each new token lies in its own sequence's tail block, as paged serving allocates them).  A
 * context length <= 0 appends nothing.  One above max_blocks_per_sequence * block_size puts the new
 * token outside the table: it is neither stored nor attended, and the call attends over the
 * table's max_blocks_per_sequence * block_size tokens exactly as rk_pa_decode does (the decode
 * clamps the context length there).  A new token whose block id is outside [0, num_blocks) is not
 * stored and is masked, as the append and the decode each treat it.
 *
 * counters/counter_words: NULL for the two-launch form (partition kernel, then the reduce kernel
 * when a sequence can span several partitions), or the counters of rk_pa_decode_fused for the
 * single-launch form.  variant: RK_PA_VARIANT_MFMA or RK_PA_VARIANT_MFMA_QK (RK_ERR_UNSUPPORTED otherwise).
 */
int rk_pa_decode_append(const void* query, const void* new_key, const void* new_value, void* key_cache,
                        void* value_cache, const void* block_tables, const void* context_lengths,
                        void* output, void* workspace, size_t workspace_bytes, uint32_t* counters,
                        size_t counter_words, int64_t batch, int64_t query_heads, int64_t kv_heads,
                        int64_t head_dim, int64_t num_blocks, int64_t block_size,
                        int64_t max_blocks_per_sequence, float scale, int dtype, int index_dtype,
                        int64_t partition_tokens, int variant, void* stream);

/*
 * Allocation-free decode.  No counterpart in the reference: it exists for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as rk_pa_decode (the same two launches, so the
 * output is bit-identical), minus the workspace: the split-K records go to a device array the
 * library holds, RK_PA_NOALLOC_SCRATCH_BYTES bytes per GPU, from the first call on that GPU until
 * the process ends.  The call makes no hipMalloc/hipFree or other allocating call; the first call
 * on a device looks up that device's array address once.
 *
 * A shape whose rk_pa_decode_workspace_bytes exceeds RK_PA_NOALLOC_SCRATCH_BYTES is rejected with
 * RK_ERR_WORKSPACE before anything is launched (a larger partition_tokens needs fewer records).
 * The stream must belong to the current device (RK_ERR_INVALID_ARGUMENT otherwise).
 *
 * Every call on one GPU shares that GPU's array: calls that may overlap in time on one GPU
 * (different streams, or different host threads without stream ordering) race on it and must be
 * serialised by the caller.  Calls in one stream's order are safe.
 */
#define RK_PA_NOALLOC_SCRATCH_BYTES (32u * 1024u * 1024u)
int rk_pa_decode_noalloc(const void* query, const void* key_cache, const void* value_cache,
                         const void* block_tables, const void* context_lengths, void* output,
                         int64_t batch, int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                         int64_t num_blocks, int64_t block_size, int64_t max_blocks_per_sequence,
                         float scale, int dtype, int index_dtype, int64_t partition_tokens,
                         int variant, void* stream);

/* Text describing the last non-RK_OK status returned on the calling thread. */
const char* rk_pa_last_error(void);

/* Library version and target, e.g. "rk_pa_gfx950 1.0.0 (gfx950, wave64)". */
const char* rk_pa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* RK_PAGED_ATTENTION_H */
