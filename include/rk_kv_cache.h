/*
 * rk_kv_cache.h -- C ABI of the gfx950 (MI355X) paged KV-cache library (librk_kv_gfx950.so).
 *
 * Writes new tokens' K/V rows into, and copies whole blocks within, the same paged cache that
 * rk_paged_attention.h reads.  Plain
 * device pointers and int64_t sizes, no torch types; calls are asynchronous on the given HIP stream,
 * never read device memory from the host and can be captured into a HIP graph.
 *
 * Reference interface each entry point replaces (zihaomu/radeon-kernels):
 *   rk_kv_cache_append -> benchmarks/kv_cache/native_kv_cache.hip:22-51 (append_kernel), launched
 *                         by append_impl (:154-189) behind the bindings append_{scalar,vec4,vec8}
 *                         (:259-283, :303-306), reached from src/radeon_kernels/providers/native.py:25
 *                         with the arguments built at src/radeon_kernels/ops/kv_cache/api.py:121.
 *   rk_kv_cache_copy   -> benchmarks/kv_cache/native_kv_cache.hip:54-80 (copy_kernel), launched by
 *                         copy_impl (:231-257) behind the bindings copy_{scalar,vec4,vec8}
 *                         (:286-298, :307-309), reached from src/radeon_kernels/providers/native.py:25
 *                         with the arguments built at src/radeon_kernels/ops/kv_cache/api.py:172.
 *   rk_kv_last_error, rk_kv_version
 *                      -> error text that TORCH_CHECK carried in the reference (:83-104,168-187).
 *
 * Layouts (row-major, contiguous; contracts/kv_cache_append-1.0.json:5-18):
 *   key, value        [tokens, kv_heads, head_dim]                   fp16 | bf16
 *   key_cache         [num_blocks, block_size, kv_heads, head_dim]   same dtype, written in place
 *   value_cache       [num_blocks, block_size, kv_heads, head_dim]   same dtype, written in place
 *   slot_mapping      [tokens]                                       int32 | int64
 *
 * Semantics (src/radeon_kernels/ops/kv_cache/reference.py:6-20): token t's K row (kv_heads x
 * head_dim elements) is copied to key_cache slot slot_mapping[t] (block = slot / block_size, offset =
 * slot % block_size), likewise V.  Bit-exact copies.  Slots must be unique; a slot outside
 * [0, num_blocks * block_size) is skipped (the token is not written).
 */
#ifndef RK_KV_CACHE_H
#define RK_KV_CACHE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (same values as rk_paged_attention.h). */
#define RK_KV_OK 0
#define RK_KV_ERR_INVALID_ARGUMENT 1 /* shapes, pointers or enum values violate the contract */
#define RK_KV_ERR_UNSUPPORTED 2      /* valid for the operator but not for this kernel */
#define RK_KV_ERR_LAUNCH 4           /* the HIP runtime rejected a launch */

/* Element types (same values as rk_paged_attention.h). */
#define RK_KV_DTYPE_FP16 0
#define RK_KV_DTYPE_BF16 1
#define RK_KV_INDEX_INT32 0
#define RK_KV_INDEX_INT64 1

/*
 * Append `tokens` K/V rows to the paged caches.  Supported by this library: all pointers 16-byte
 * aligned and kv_heads * head_dim * 2 a multiple of 16 bytes (whole 16-byte chunks per row);
 * tokens * kv_heads * head_dim < 2^31.
 */
int rk_kv_cache_append(const void* key, const void* value, void* key_cache, void* value_cache,
                       const void* slot_mapping, int64_t tokens, int64_t kv_heads,
                       int64_t head_dim, int64_t num_blocks, int64_t block_size, int dtype,
                       int index_dtype, void* stream);

/*
 * Copy cache blocks: for each of the `pairs` rows (source, destination) of block_mapping
 * [pairs, 2] (int32 or int64), block `source` of both caches is copied to block `destination`
 * (reference.py:23-38).  Destinations must be unique and disjoint from the sources
 * (contracts/kv_cache_copy-1.0.json:17); every copy then reads the pre-call contents.  A pair with
 * a block id outside [0, num_blocks) is skipped.  Supported: caches 16-byte aligned and
 * block_size * kv_heads * head_dim * 2 a multiple of 16 bytes.
 */
int rk_kv_cache_copy(void* key_cache, void* value_cache, const void* block_mapping, int64_t pairs,
                     int64_t num_blocks, int64_t block_size, int64_t kv_heads, int64_t head_dim,
                     int dtype, int index_dtype, void* stream);

/* Text describing the last non-RK_KV_OK status returned on the calling thread. */
const char* rk_kv_last_error(void);

/* Library version and target, e.g. "rk_kv_gfx950 1.0.0 (gfx950, wave64)". */
const char* rk_kv_version(void);

#ifdef __cplusplus
}
#endif

#endif /* RK_KV_CACHE_H */
