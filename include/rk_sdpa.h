/*
 * rk_sdpa.h -- C ABI of the gfx950 (MI355X) scaled dot-product self-attention library.
 *
 * Library: librk_sdpa_gfx950.so (hand-written HIP for CDNA4, wave64).  Every tensor is a device
 * pointer to a dense, contiguous buffer; the call is asynchronous on the given HIP stream, needs no
 * workspace and never reads device memory from the host, so it can be captured into a HIP graph.
 *
 * Reference interface it replaces (zihaomu/radeon-kernels): the native entrypoint that a dispatch
 * entry of sdpa 1.0 would name, called as entrypoint(query, key, value, is_causal, scale)
 * (src/radeon_kernels/ops/sdpa/api.py:94-105 builds exactly these native arguments; the reference
 * publishes no such kernel -- dispatch/sdpa-1.0.json has no entries -- so its declared fallback,
 * torch scaled_dot_product_attention, src/radeon_kernels/ops/sdpa/reference.py:41-58, is the
 * behaviour replaced).
 *
 * Layouts (row-major, contiguous), contracts/sdpa-1.0.json:5-12:
 *   query   [batch, query_heads, sequence, head_dim]   fp16 | bf16
 *   key     [batch, kv_heads,    sequence, head_dim]   dtype of query
 *   value   [batch, kv_heads,    sequence, head_dim]   dtype of query
 *   output  [batch, query_heads, sequence, head_dim]   dtype of query
 *
 * Semantics (src/radeon_kernels/ops/sdpa/reference.py:13-38): query head h attends with KV head
 * h / (query_heads / kv_heads); scores q . k * scale; with is_causal, query i sees keys j <= i;
 * softmax and both contractions accumulate in fp32 (the probabilities enter the second contraction
 * rounded to the input dtype); non-finite inputs propagate.
 */
#ifndef RK_SDPA_H
#define RK_SDPA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RK_SDPA_OK 0
#define RK_SDPA_ERR_INVALID_ARGUMENT 1 /* shapes, pointers or scalars violate the contract */
#define RK_SDPA_ERR_UNSUPPORTED 2      /* valid for the operator but not for this kernel */
#define RK_SDPA_ERR_LAUNCH 4           /* the HIP runtime rejected the launch */

#define RK_SDPA_DTYPE_FP16 0
#define RK_SDPA_DTYPE_BF16 1

/*
 * Self-attention forward pass.  head_dim in {64, 128, 256}; query_heads % kv_heads == 0;
 * is_causal 0 or 1; scale positive and finite (1/sqrt(head_dim) is the operator's default);
 * stream is a hipStream_t (NULL = the null stream).
 */
int rk_sdpa_forward(const void* query, const void* key, const void* value, void* output, int64_t batch,
                    int64_t query_heads, int64_t kv_heads, int64_t sequence, int64_t head_dim, int is_causal,
                    float scale, int dtype, void* stream);

/* Text describing the last non-RK_SDPA_OK status returned on the calling thread. */
const char* rk_sdpa_last_error(void);

/* Library version and target, e.g. "rk_sdpa_gfx950 1.0.0 (gfx950, wave64)". */
const char* rk_sdpa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* RK_SDPA_H */
