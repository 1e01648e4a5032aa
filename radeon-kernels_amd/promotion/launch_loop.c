/*
 * Launch loops for the promotion timing (promotion/evaluate.py).
 *
 * Each function calls one of the product's C-ABI entry points n times in a row, walking input copies
 * first, first + 1, ... (mod copies) for the cache arguments, and returns the first non-zero status
 * (0 when every call succeeded).  The entry point is passed as a function pointer taken from the
 * product library, so this file links against nothing.  A timing batch of microsecond-scale calls
 * is then paced by the GPU and the HIP launch path, as it is in a C or C++ serving loop, rather than
 * by one interpreter-level foreign call per launch.
 */
#include <stddef.h>
#include <stdint.h>

typedef int (*decode_fn)(const void*, const void*, const void*, const void*, const void*, void*, void*, size_t,
                         int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, float, int, int,
                         int64_t, int, void*);
typedef int (*decode_fused_fn)(const void*, const void*, const void*, const void*, const void*, void*, void*,
                               size_t, uint32_t*, size_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                               int64_t, float, int, int, int64_t, int, void*);
typedef int (*append_fn)(const void*, const void*, void*, void*, const void*, int64_t, int64_t, int64_t, int64_t,
                         int64_t, int, int, void*);
typedef int (*copy_fn)(void*, void*, const void*, int64_t, int64_t, int64_t, int64_t, int64_t, int, int, void*);
typedef int (*sdpa_fn)(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t, int64_t,
                       int, float, int, void*);

/* rk_pa_decode (counters == NULL) or rk_pa_decode_fused. */
int loop_decode(void* fn, int64_t n, int64_t first, int64_t copies, const void* query, void* const* key_caches,
                void* const* value_caches, const void* block_tables, const void* context_lengths, void* output,
                void* workspace, size_t workspace_bytes, uint32_t* counters, size_t counter_words, int64_t batch,
                int64_t query_heads, int64_t kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                int64_t max_blocks, float scale, int dtype, int index_dtype, int64_t partition_tokens,
                int variant, void* stream) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t c = (first + i) % copies;
    const int status =
        counters == NULL
            ? ((decode_fn)fn)(query, key_caches[c], value_caches[c], block_tables, context_lengths, output,
                              workspace, workspace_bytes, batch, query_heads, kv_heads, head_dim, num_blocks,
                              block_size, max_blocks, scale, dtype, index_dtype, partition_tokens, variant, stream)
            : ((decode_fused_fn)fn)(query, key_caches[c], value_caches[c], block_tables, context_lengths, output,
                                    workspace, workspace_bytes, counters, counter_words, batch, query_heads,
                                    kv_heads, head_dim, num_blocks, block_size, max_blocks, scale, dtype,
                                    index_dtype, partition_tokens, variant, stream);
    if (status != 0) return status;
  }
  return 0;
}

/* rk_kv_cache_append. */
int loop_append(void* fn, int64_t n, int64_t first, int64_t copies, const void* key, const void* value,
                void* const* key_caches, void* const* value_caches, const void* slot_mapping, int64_t tokens,
                int64_t kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size, int dtype,
                int index_dtype, void* stream) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t c = (first + i) % copies;
    const int status = ((append_fn)fn)(key, value, key_caches[c], value_caches[c], slot_mapping, tokens, kv_heads,
                                       head_dim, num_blocks, block_size, dtype, index_dtype, stream);
    if (status != 0) return status;
  }
  return 0;
}

/* rk_kv_cache_copy. */
int loop_copy(void* fn, int64_t n, int64_t first, int64_t copies, void* const* key_caches,
              void* const* value_caches, const void* block_mapping, int64_t pairs, int64_t num_blocks,
              int64_t block_size, int64_t kv_heads, int64_t head_dim, int dtype, int index_dtype, void* stream) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t c = (first + i) % copies;
    const int status = ((copy_fn)fn)(key_caches[c], value_caches[c], block_mapping, pairs, num_blocks, block_size,
                                     kv_heads, head_dim, dtype, index_dtype, stream);
    if (status != 0) return status;
  }
  return 0;
}

/* rk_sdpa_forward (no rotation: one input set). */
int loop_sdpa(void* fn, int64_t n, const void* query, const void* key, const void* value, void* output,
              int64_t batch, int64_t query_heads, int64_t kv_heads, int64_t sequence, int64_t head_dim,
              int is_causal, float scale, int dtype, void* stream) {
  for (int64_t i = 0; i < n; ++i) {
    const int status = ((sdpa_fn)fn)(query, key, value, output, batch, query_heads, kv_heads, sequence, head_dim,
                                     is_causal, scale, dtype, stream);
    if (status != 0) return status;
  }
  return 0;
}
