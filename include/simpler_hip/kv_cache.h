/* KV-cache append and the fused decode prelude (q/k RMS norm + RoPE + append)
 * on gfx950 (MI355X).
 *
 * These replace the step before paged-attention decode in simpler's Qwen3
 * decode layer: the current token's K/V written into the paged BSND pool at
 * slot_mapping (simpler_setup/goldens/qwen3_14b_decode.py:106-115,261-269),
 * and the prelude that produces them and the query
 * (qwen3_14b_decode.py:207-226): per-head RMS norm with a learned weight,
 * half-split RoPE at position seq_len - 1, bf16 rounding. In the reference the
 * prelude and the cache write are phase 0 of the fused attention task
 * (examples/a2a3/tensormap_and_ringbuffer/qwen3_14b_decode/kernels/vendor/
 * paged_attention_cce/kernel/fai_body.hpp:199-230, rope_qkv with
 * slot_mapping, k_cache, v_cache); here they are their own launches on the
 * caller's stream, ahead of simpler_hip_pa_decode.
 *
 * All pointers are device pointers; strides are in elements; caches are
 * [num_blocks, block_size, num_kv_heads, head_dim] bf16 with unit stride in the
 * head dim. A slot is physical_block * block_size + offset_in_block. Negative
 * slots are skipped (padding tokens). Slots past the pool and positions
 * outside the RoPE table are skipped and counted in *error_count when that
 * optional device counter is given. Both calls allocate nothing and are
 * asynchronous on `stream` (a hipStream_t, NULL = default stream).
 */
#ifndef SIMPLER_HIP_KV_CACHE_H
#define SIMPLER_HIP_KV_CACHE_H

#include <stdint.h>

#include "simpler_hip/pa_decode.h" /* error codes */

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

typedef struct SimplerHipKvAppendArgs {
    const void *key;             /* [num_tokens, num_kv_heads, head_dim_k] bf16 */
    const void *value;           /* [num_tokens, num_kv_heads, head_dim_v] bf16; NULL: K only (MLA latent) */
    const int32_t *slot_mapping; /* [num_tokens] */
    void *key_cache;
    void *value_cache; /* NULL when value is NULL */
    int32_t *error_count;
    int64_t key_token_stride, key_head_stride;
    int64_t value_token_stride, value_head_stride;
    int64_t k_block_stride, k_token_stride, k_head_stride;
    int64_t v_block_stride, v_token_stride, v_head_stride;
    int32_t num_tokens, num_kv_heads, head_dim_k, head_dim_v, block_size, num_blocks;
} SimplerHipKvAppendArgs;

/* Write each token's K (and V) rows into the paged caches at its slot
 * (qwen3_14b_decode.py:261-269). head dims: multiples of 8, at most 1024;
 * 16-byte aligned rows. */
int simpler_hip_kv_append(const SimplerHipKvAppendArgs *args, void *stream);

typedef struct SimplerHipQkNormRopeAppendArgs {
    const float *q_proj;         /* [batch, num_heads * head_dim] fp32 */
    const float *k_proj;         /* [batch, num_kv_heads * head_dim] fp32 */
    const float *v_proj;         /* [batch, num_kv_heads * head_dim] fp32 */
    const float *inv_rms;        /* [batch] fp32: rsqrt(mean(h^2) + eps) of the hidden state */
    const float *q_norm_weight;  /* [head_dim] fp32 */
    const float *k_norm_weight;  /* [head_dim] fp32 */
    const float *rope_cos;       /* [max_position, head_dim] fp32 */
    const float *rope_sin;       /* [max_position, head_dim] fp32 */
    const int32_t *seq_lens;     /* [batch]: the token's position is seq_len - 1 */
    const int32_t *slot_mapping; /* [batch] */
    void *q_out;                 /* [batch, num_heads, head_dim] bf16 */
    void *key_cache;
    void *value_cache;
    int32_t *error_count;
    int64_t k_block_stride, k_token_stride, k_head_stride;
    int64_t v_block_stride, v_token_stride, v_head_stride;
    int32_t batch, num_heads, num_kv_heads, head_dim, block_size, num_blocks, max_position;
    float eps;
} SimplerHipQkNormRopeAppendArgs;

/* q = rope(rmsnorm(q_proj * inv_rms) * q_norm_weight), k likewise with
 * k_norm_weight, v = v_proj * inv_rms, all rounded to bf16; q to q_out, k and
 * v into the caches at slot_mapping (qwen3_14b_decode.py:207-226,261-269).
 * head_dim even, at most 1024. A token whose position is outside the RoPE
 * table gets a zero q and no cache write. */
int simpler_hip_qk_norm_rope_append(const SimplerHipQkNormRopeAppendArgs *args, void *stream);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* SIMPLER_HIP_KV_CACHE_H */
