/*
 * simpler_hip — paged-attention decode entry points of libsimpler_hip.so.
 *
 * These replace the work that simpler's orchestration function
 * `aicpu_orchestration_entry` submits as four AICore tasks (QK, SF, PV, UP)
 * per KV block (reference: examples/a2a3/tensormap_and_ringbuffer/
 * paged_attention/kernels/orchestration/paged_attention_orch.cpp:77-291).
 * The argument meaning follows that function's 7-argument contract
 * (:94-102): query, key_cache, value_cache, block_table, context_lens, out,
 * scale. Here the whole chain is one fused split-K gfx950 kernel.
 *
 * Plain C ABI: device pointers, sizes and an opaque HIP stream (hipStream_t
 * passed as void*; NULL = the null stream). No torch types.
 */
#ifndef SIMPLER_HIP_PA_DECODE_H
#define SIMPLER_HIP_PA_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

/* Error codes (0 = success, negative = error; same convention as the reference
 * C API, src/common/worker/pto_runtime_c_api.h:50,73-83). */
enum {
    SIMPLER_HIP_OK = 0,
    SIMPLER_HIP_ERR_INVALID = -1,     /* bad shape / dtype / argument          */
    SIMPLER_HIP_ERR_UNSUPPORTED = -2, /* == PTO_RUNTIME_ERR_UNSUPPORTED         */
    SIMPLER_HIP_ERR_WORKSPACE = -4,   /* workspace missing or too small         */
    SIMPLER_HIP_ERR_LAUNCH = -5,      /* HIP launch / runtime failure           */
    SIMPLER_HIP_ERR_BAD_BLOCK = -6,   /* block_table entry outside the KV pool  */
    SIMPLER_HIP_ERR_BAD_LENGTH = -7,  /* context_lens entry outside [0, max_blocks_per_seq*block_size],
                                         or (causal) shorter than q_len           */
};

/* Output dtypes, using the reference's DataType codes
 * (src/common/task_interface/data_type.h:47-67). */
enum { SIMPLER_HIP_DT_FLOAT32 = 0, SIMPLER_HIP_DT_FLOAT16 = 1, SIMPLER_HIP_DT_BFLOAT16 = 6 };

/* Element formats of the query and KV caches. BF16: bf16 query and caches.
 * FP8_E4M3: bf16 query, OCP E4M3FN cache bytes (the reference's DataType
 * FP8E4M3FN, data_type.h:63) with one fp32 scale per (physical block, kv
 * head); head dims 128, block sizes 16/32/64/128, GQA path (not MLA).
 * FP16: fp16 query and caches (the dtype of the reference's GQA scene cases,
 * tests/st/a2a3/tensormap_and_ringbuffer/spmd_paged_attention_highperf/
 * test_spmd_paged_attention_highperf.py:170-232); p is rounded to fp16 as
 * the golden rounds it to the input dtype; GQA path (not MLA). */
enum { SIMPLER_HIP_KV_BF16 = 0, SIMPLER_HIP_KV_FP8_E4M3 = 1, SIMPLER_HIP_KV_FP16 = 2 };

/*
 * One paged-attention decode call. All pointers are device pointers.
 *
 * query        bf16 (fp16 with kv_format FP16) [batch, q_len, num_heads, head_dim_k]
 *              (q_len = 1: [batch, num_heads, Dk])
 * key_cache    bf16 (fp8 or fp16, see kv_format), element (blk, t, kvh, d) at
 *              blk*k_block_stride + t*k_token_stride + kvh*k_head_stride + d
 *              (contiguous BSND [num_blocks, block_size, kv_heads, Dk]:
 *               strides BS*Hkv*Dk, Hkv*Dk, Dk)
 * value_cache  same element type, same addressing with the v_* strides and Dv columns.
 *              MLA: value_cache == key_cache with the K strides and Dv <= Dk
 *              (V is the first Dv columns of K).
 * block_table  int32 [batch, max_blocks_per_seq], entries in [0, num_blocks)
 * context_lens int32 [batch], 0 <= len <= max_blocks_per_seq*block_size
 * out          [batch, q_len, num_heads, Dv] of out_dtype: FLOAT32 or BFLOAT16
 *              (bf16 and fp8 caches), FLOAT32 or FLOAT16 (fp16 caches)
 * scale        softmax scale applied to q.k in fp32
 * causal       q_len > 1 only: query token i sees context_len - (q_len-1-i) tokens
 */
typedef struct SimplerHipPaDecodeArgs {
    const void *query;
    const void *key_cache;
    const void *value_cache;
    const int32_t *block_table;
    const int32_t *context_lens;
    void *out;
    int64_t k_block_stride, k_token_stride, k_head_stride;
    int64_t v_block_stride, v_token_stride, v_head_stride;
    int32_t batch;
    int32_t q_len;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim_k;
    int32_t head_dim_v;
    int32_t block_size;
    int32_t max_blocks_per_seq;
    int32_t num_blocks;
    int32_t out_dtype;
    float scale;
    int32_t causal;
    /* 0 = one worker wavefront per wave slot of the device; > 0 forces the
     * number of workers the (tile, KV block) work list is divided among. */
    int32_t num_workers;
    /* SIMPLER_HIP_KV_BF16 (0), SIMPLER_HIP_KV_FP8_E4M3 (1) or SIMPLER_HIP_KV_FP16 (2). */
    int32_t kv_format;
    /* kv_format FP8_E4M3 only: fp32 [num_blocks, num_kv_heads] dequantisation
     * scales; cache element (blk, t, kvh, d) stands for
     * fp8_e4m3fn(byte) * scale[blk * num_kv_heads + kvh]. NULL otherwise. */
    const float *k_scale;
    const float *v_scale;
} SimplerHipPaDecodeArgs;

/* Bytes of device workspace simpler_hip_pa_decode needs for these args
 * (error word + two partial-result slots per worker). Depends on the current
 * device (its wave-slot count) when num_workers is 0. */
size_t simpler_hip_pa_decode_workspace_size(const SimplerHipPaDecodeArgs *args);

/* Zero a freshly allocated workspace (the error word must start at zero).
 * Enqueued on `stream`. */
int simpler_hip_pa_decode_workspace_init(void *workspace, size_t workspace_bytes, void *stream);

/*
 * Enqueue the decode on `stream`: the fused kernel (one wavefront per worker,
 * each over an equal slice of the flattened (tile, KV block) work), then the
 * small kernel that merges tiles cut between workers. `workspace` must be at
 * least simpler_hip_pa_decode_workspace_size(args) bytes, 256-byte aligned,
 * initialised once with simpler_hip_pa_decode_workspace_init, and not shared by
 * calls that may run concurrently. Returns 0 or a negative SIMPLER_HIP_ERR_*
 * code (shape and dtype checks happen on the host before anything is launched).
 */
int simpler_hip_pa_decode(const SimplerHipPaDecodeArgs *args, void *workspace, size_t workspace_bytes, void *stream);

/* The two kernels of simpler_hip_pa_decode, separately (measurement: lets a
 * caller put timing events between them). Running MAIN then MERGE on one
 * stream is exactly simpler_hip_pa_decode; MERGE reads what MAIN wrote to the
 * workspace, so it must follow a MAIN with the same args and workspace. */
enum { SIMPLER_HIP_PHASE_MAIN = 1, SIMPLER_HIP_PHASE_MERGE = 2 };
int simpler_hip_pa_decode_phase(const SimplerHipPaDecodeArgs *args, void *workspace, size_t workspace_bytes,
                                void *stream, int phases);

/* After the stream has completed: returns SIMPLER_HIP_ERR_BAD_BLOCK if any
 * launch since the last check met an out-of-pool block_table entry (such
 * blocks are skipped, never dereferenced), else SIMPLER_HIP_ERR_BAD_LENGTH if
 * one read a context_lens entry below 0, above max_blocks_per_seq*block_size,
 * or (causal, or with the fused append) below q_len (the kernels then use the length clamped into
 * [0, max_blocks_per_seq*block_size]), else 0. Clears the flags. Synchronous. */
int simpler_hip_pa_decode_check(void *workspace, size_t workspace_bytes, void *stream);

/*
 * simpler_hip_pa_decode for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Instead of a caller workspace
 * it uses a fixed device array of SIMPLER_HIP_PA_NOALLOC_SCRATCH_BYTES inside
 * this library, one per GPU, held until the process ends; it calls no
 * hipMalloc/hipFree. Same arguments, kernels and results as
 * simpler_hip_pa_decode on the same args. Returns SIMPLER_HIP_ERR_WORKSPACE
 * (and says so on stderr) when the decode's plan needs more scratch than that
 * (possible only with a forced num_workers). Calls on one GPU share its array:
 * calls that may overlap on one GPU (different streams) race and must not be
 * made. Out-of-pool block ids and bad lengths found by the kernels are handled
 * as in simpler_hip_pa_decode (skipped / clamped) but not reported: there is
 * no workspace to pass to simpler_hip_pa_decode_check.
 */
#define SIMPLER_HIP_PA_NOALLOC_SCRATCH_BYTES (136u << 20)
int simpler_hip_pa_decode_noalloc(const SimplerHipPaDecodeArgs *args, void *stream);

/*
 * KV-cache append fused into the decode: writes each sequence's new tokens
 * into the paged caches and attends over the context that includes them, in
 * the decode's two launches. Replaces the reference's separate append (the
 * slot_mapping scatter of simpler_setup/goldens/qwen3_14b_decode.py:106-115,
 * 261-269, which its fused attention task runs as phase 0,
 * examples/a2a3/tensormap_and_ringbuffer/qwen3_14b_decode/kernels/vendor/
 * paged_attention_cce/kernel/fai_body.hpp:199-230) followed by the decode.
 *
 * key_new    [batch, q_len, num_kv_heads, head_dim_k], the caches' element
 *            type (bf16 or fp16), contiguous, 16-byte aligned
 * value_new  [batch, q_len, num_kv_heads, head_dim_v], same; NULL for MLA
 *            (value_cache == key_cache: V is the first head_dim_v dims of the
 *            K row written)
 * The q_len new tokens of sequence b are its last positions: with len =
 * context_lens[b] (which counts them), token j goes to position
 * p = len - q_len + j, i.e. row p % block_size of block
 * block_table[b][p / block_size] -- the slot the reference derives from the
 * block table and seq_len (qwen3_14b_decode.py:106-115). Results and cache
 * contents are those of simpler_hip_kv_append with that slot mapping followed
 * by simpler_hip_pa_decode. q_len <= 16; bf16 and fp16 caches (not fp8).
 * The append is fused into the decode's two launches where each worker runs
 * one row tile; where the decode gives a worker several row tiles (GQA with
 * more than 16 query rows per kv head) and for MLA, it runs as a launch of
 * its own ahead of them, which measured faster there. Both forms leave the
 * same cache contents.
 * Same workspace as simpler_hip_pa_decode for these args. A length below
 * q_len or above max_blocks_per_seq*block_size is reported by
 * simpler_hip_pa_decode_check as BAD_LENGTH: the new tokens are still placed
 * by the raw length, only those at positions in
 * [0, max_blocks_per_seq*block_size) are written (the others are dropped and
 * no other cache row changes), and the decode attends over the length clamped
 * into that range. New tokens in out-of-pool blocks are neither read nor
 * written (BAD_BLOCK).
 */
int simpler_hip_pa_decode_append(const SimplerHipPaDecodeArgs *args, const void *key_new, const void *value_new,
                                 void *workspace, size_t workspace_bytes, void *stream);

/*
 * The decode prelude, the KV append and the decode in one call: the query and
 * the new tokens' K/V are computed from the fp32 projections as
 * simpler_hip_qk_norm_rope_append (include/simpler_hip/kv_cache.h) computes
 * them -- q/k = RoPE(RMSnorm(proj * inv_rms) * weight), half-split RoPE,
 * v = proj * inv_rms, all rounded to bf16 -- the new K/V are written into the
 * caches at each sequence's last q_len positions (the slots the block table
 * gives, as for simpler_hip_pa_decode_append), and the decode attends over
 * them. Replaces the reference's prelude + append + attention of one decode
 * layer (simpler_setup/goldens/qwen3_14b_decode.py:207-226, 261-269, then the
 * paged attention; in the reference the prelude and the cache write are
 * phase 0 of the fused attention task, paged_attention_cce/kernel/
 * fai_body.hpp:199-230). Three launches on `stream`: the prelude (its query
 * rows into the workspace), then the decode's two. Results and cache
 * contents equal, bit for bit, simpler_hip_qk_norm_rope_append per token
 * (position context_lens[b] - q_len + i, slot from the block table) followed
 * by simpler_hip_pa_decode on its query.
 *
 * args: as for simpler_hip_pa_decode_append, with bf16 caches (kv_format
 * BF16), head_dim_k = head_dim_v = 128, a GQA cache (not MLA), q_len <= 16;
 * args->query is not read (it may be NULL). Workspace: at least
 * simpler_hip_pa_decode_prelude_workspace_size(args) bytes (the decode's, then
 * the bf16 query rows), otherwise as for simpler_hip_pa_decode.
 * A sequence whose length is below q_len or above max_position is reported by
 * simpler_hip_pa_decode_check as BAD_LENGTH; its tokens outside the RoPE table
 * get a zero query row and do not write cache rows.
 */
typedef struct SimplerHipDecodePreludeArgs {
    const float *q_proj;        /* [batch, q_len, num_heads, 128] fp32 */
    const float *k_proj;        /* [batch, q_len, num_kv_heads, 128] fp32 */
    const float *v_proj;        /* [batch, q_len, num_kv_heads, 128] fp32 */
    const float *inv_rms;       /* [batch, q_len] fp32: rsqrt(mean(h^2) + eps) of the hidden state */
    const float *q_norm_weight; /* [128] fp32 */
    const float *k_norm_weight; /* [128] fp32 */
    const float *rope_cos;      /* [max_position, 128] fp32 */
    const float *rope_sin;      /* [max_position, 128] fp32 */
    int32_t max_position;
    float eps;
} SimplerHipDecodePreludeArgs;

int simpler_hip_pa_decode_prelude(const SimplerHipPaDecodeArgs *args, const SimplerHipDecodePreludeArgs *prelude,
                                  void *workspace, size_t workspace_bytes, void *stream);
/* Bytes of workspace simpler_hip_pa_decode_prelude needs for these args (0 if
 * unsupported or invalid). */
size_t simpler_hip_pa_decode_prelude_workspace_size(const SimplerHipPaDecodeArgs *args);

/* Measurement helpers: name of the main kernel the args select, and the
 * number of worker wavefronts a launch uses. */
const char *simpler_hip_pa_decode_kernel_name(const SimplerHipPaDecodeArgs *args);
int simpler_hip_pa_decode_plan(const SimplerHipPaDecodeArgs *args, int32_t *num_workers);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* SIMPLER_HIP_PA_DECODE_H */
