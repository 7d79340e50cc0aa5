// KV-cache append and the fused decode prelude (q/k RMS norm + RoPE + append)
// for gfx950 (MI355X).
//
// Reference: simpler's Qwen3 decode golden, simpler_setup/goldens/
// qwen3_14b_decode.py — slot mapping :106-115, prelude :207-226 (q/k scaled by
// the hidden state's inverse RMS, per-head RMS norm with eps and a weight,
// half-split RoPE :99-103 at position seq_len - 1, bf16 rounding), cache write
// :261-269 (row slot * kv_heads + kv_head of the flat BSND pool). In the
// reference these run as phase 0 of the fused attention task
// (kernels/vendor/paged_attention_cce/kernel/fai_body.hpp:199-230).
//
// Both also run in a paged form for the decode entries of pa_decode.h
// (simpler_hip_pa_decode_append / _prelude): token t of the launch is position
// context_lens[b] - q_len + j of sequence b = t / q_len (j = t % q_len), its
// slot the block-table row's, as the reference derives it
// (qwen3_14b_decode.py:106-115).
//
// Both kernels are HBM- or launch-bound byte movers:
//   kv_append_kernel           one workgroup per token: 16-byte vector copies of
//                              its K (and V) rows.
//   qk_norm_rope_append_kernel one wave per (token, head): lane i holds elements
//                              i and i + D/2 (the two RoPE halves), so the
//                              rotation needs no cross-lane traffic; the sum of
//                              squares is a wave reduction.
// The fp32 arithmetic follows the golden's operation order with no fused
// multiply-adds (products rounded before the sum, as torch evaluates
// `lo * cos - hi * sin`), correctly rounded sqrt and division. The sum of
// squares is reduced in a different order than torch's mean, so a result can
// differ from the golden by one bf16 rounding step.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "simpler_hip/kv_cache.h"
#include "pa_decode_internal.h"

namespace simpler_hip_kv {
namespace {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxHeadDim = 1024;

// The paged form's token -> (position, slot) inputs; block_table null: the
// caller's slot mapping (and seq_lens) instead.
struct Paged {
    const int32_t *block_table, *context_lens;
    unsigned *error_flag;  // the decode workspace's error word
    unsigned bad_length;   // its bit for a length below q_len (or a position outside the RoPE table)
    int32_t q_len, max_blocks;
};

struct AppendParams {
    const uint16_t *key, *value;
    const int32_t *slot;
    uint16_t *kc, *vc;
    int32_t *err;
    int64_t key_ts, key_hs, val_ts, val_hs;
    int64_t k_bs, k_ts, k_hs, v_bs, v_ts, v_hs;
    int32_t num_tokens, hkv, dk, dv, block_size, num_blocks;
    Paged pg;
};

__device__ __forceinline__ bool slot_ok(int slot, int32_t num_blocks, int32_t block_size, int32_t *err) {
    if (slot < 0) return false;  // padding token
    if ((int64_t)slot >= (int64_t)num_blocks * block_size) {
        if (threadIdx.x == 0 && err) atomicAdd(err, 1);
        return false;
    }
    return true;
}

// Paged form: position and slot of launch token t, or slot -1 where the
// token is not written: a position below 0 (a length below q_len, reported
// by the caller of this), one past the block-table row (a length the decode
// reports), or an out-of-pool block (reported when the decode reads it).
__device__ __forceinline__ int paged_slot(const Paged &G, const int t, const int32_t block_size,
                                          const int32_t num_blocks, int *pos) {
    const int b = t / G.q_len;
    const int p = G.context_lens[b] - G.q_len + (t - b * G.q_len);
    *pos = p;
    if (p < 0 || p >= G.max_blocks * block_size) return -1;
    const int phys = G.block_table[(int64_t)b * G.max_blocks + p / block_size];
    if ((unsigned)phys >= (unsigned)num_blocks) return -1;
    return phys * block_size + p % block_size;
}

__global__ void __launch_bounds__(kThreads) kv_append_kernel(const AppendParams P) {
    const int t = blockIdx.x;
    int pos = 0;
    const int slot = P.pg.block_table ? paged_slot(P.pg, t, P.block_size, P.num_blocks, &pos) : P.slot[t];
    if (pos < 0 && threadIdx.x == 0) atomicOr(P.pg.error_flag, P.pg.bad_length);  // paged form only
    if (!slot_ok(slot, P.num_blocks, P.block_size, P.err)) return;
    const int blk = slot / P.block_size, off = slot - blk * P.block_size;
    const int kch = P.dk / 8;
    for (int i = threadIdx.x; i < P.hkv * kch; i += kThreads) {
        const int h = i / kch, c = i - h * kch;
        const u32x4_t v = *reinterpret_cast<const u32x4_t *>(P.key + t * P.key_ts + h * P.key_hs + 8 * c);
        *reinterpret_cast<u32x4_t *>(P.kc + blk * P.k_bs + off * P.k_ts + h * P.k_hs + 8 * c) = v;
    }
    if (!P.value) return;
    const int vch = P.dv / 8;
    for (int i = threadIdx.x; i < P.hkv * vch; i += kThreads) {
        const int h = i / vch, c = i - h * vch;
        const u32x4_t v = *reinterpret_cast<const u32x4_t *>(P.value + t * P.val_ts + h * P.val_hs + 8 * c);
        *reinterpret_cast<u32x4_t *>(P.vc + blk * P.v_bs + off * P.v_ts + h * P.v_hs + 8 * c) = v;
    }
}

struct PreludeParams {
    const float *q_proj, *k_proj, *v_proj, *inv_rms, *q_w, *k_w, *cos, *sin;
    const int32_t *seq_lens, *slot;
    uint16_t *q_out, *kc, *vc;
    int32_t *err;
    int64_t k_bs, k_ts, k_hs, v_bs, v_ts, v_hs;
    int32_t batch, hq, hkv, d, block_size, num_blocks, max_pos;
    float eps;
    Paged pg;
};

// fp32 -> bf16, round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint16_t to_bf16(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// One wave per (token, head unit): units are the q heads, then the k heads,
// then the v heads, so every row's loads are in flight at once. DFIX: the
// head dim when fixed at compile time (128: one element of each half per
// lane), 0 for any even head dim up to kMaxHeadDim. The loads that do not
// depend on the token's position (the row, inv_rms, the norm weight) are
// issued before it is known, so the position's load and the RoPE rows' loads
// are the only ones in sequence.
template <int DFIX>
__global__ void __launch_bounds__(64) qk_norm_rope_append_kernel(const PreludeParams P) {
#pragma clang fp contract(off)
    constexpr int kPer = DFIX ? (DFIX + 127) / 128 : kMaxHeadDim / 2 / 64;  // elements of each half per lane
    const int b = blockIdx.y;
    const int u = blockIdx.x;
    const int lane = threadIdx.x;
    const int half = DFIX ? DFIX / 2 : P.d / 2;
    const bool is_q = u < P.hq, is_k = !is_q && u < P.hq + P.hkv;
    const int h = is_q ? u : (is_k ? u - P.hq : u - P.hq - P.hkv);
    const float *src = is_q ? P.q_proj + ((int64_t)b * P.hq + h) * P.d
                            : (is_k ? P.k_proj : P.v_proj) + ((int64_t)b * P.hkv + h) * P.d;
    const float *w = is_q ? P.q_w : P.k_w;
    float xl[kPer], xh[kPer], wl[kPer], wh[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = lane + 64 * j;
        xl[j] = xh[j] = wl[j] = wh[j] = 0.f;
        if (DFIX == 128 || i < half) {
            xl[j] = src[i];
            xh[j] = src[i + half];
            if (is_q || is_k) {
                wl[j] = w[i];
                wh[j] = w[i + half];
            }
        }
    }
    const float ir = P.inv_rms[b];

    int pos = 0, slot;
    if (P.pg.block_table) {
        slot = paged_slot(P.pg, b, P.block_size, P.num_blocks, &pos);
    } else {
        pos = P.seq_lens[b] - 1;
        slot = P.slot[b];
    }
    const bool pos_ok = pos >= 0 && pos < P.max_pos;
    if (!pos_ok && u == 0 && threadIdx.x == 0) {
        if (P.err) atomicAdd(P.err, 1);
        if (P.pg.error_flag) atomicOr(P.pg.error_flag, P.pg.bad_length);  // below q_len, or past the RoPE table
    }
    // count a bad slot once per token (on its first k unit)
    const bool write_kv = pos_ok && slot_ok(slot, P.num_blocks, P.block_size, u == P.hq ? P.err : nullptr);
    const int blk = write_kv ? slot / P.block_size : 0, off = write_kv ? slot - blk * P.block_size : 0;
    const float *cosr = P.cos + (int64_t)(pos_ok ? pos : 0) * P.d;
    const float *sinr = P.sin + (int64_t)(pos_ok ? pos : 0) * P.d;

    float lo[kPer], hi[kPer];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = lane + 64 * j;
        lo[j] = hi[j] = 0.f;
        if (DFIX == 128 || i < half) {
            lo[j] = xl[j] * ir;
            hi[j] = xh[j] * ir;
            ss += lo[j] * lo[j];
            ss += hi[j] * hi[j];
        }
    }
    uint16_t *dst;
    if (is_q) {
        dst = P.q_out + ((int64_t)b * P.hq + h) * P.d;
    } else {
        if (!write_kv) return;
        dst = is_k ? P.kc + blk * P.k_bs + off * P.k_ts + h * P.k_hs
                   : P.vc + blk * P.v_bs + off * P.v_ts + h * P.v_hs;
    }
    if (is_q || is_k) {
        ss = wave_sum(ss);
        const float r = __fdiv_rn(1.f, __fsqrt_rn(__fdiv_rn(ss, (float)P.d) + P.eps));
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = lane + 64 * j;
            if (DFIX != 128 && i >= half) continue;
            const float zl = (lo[j] * r) * wl[j];
            const float zh = (hi[j] * r) * wh[j];
            float ol = zl * cosr[i] - zh * sinr[i];
            float oh = zh * cosr[i + half] + zl * sinr[i + half];
            if (!pos_ok) ol = oh = 0.f;
            dst[i] = to_bf16(ol);
            dst[i + half] = to_bf16(oh);
        }
    } else {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = lane + 64 * j;
            if (DFIX != 128 && i >= half) continue;
            dst[i] = to_bf16(lo[j]);
            dst[i + half] = to_bf16(hi[j]);
        }
    }
}

// The prelude kernel for head dim d.
void launch_prelude_kernel(const PreludeParams &P, unsigned units, unsigned tokens, hipStream_t stream) {
    if (P.d == 128)
        hipLaunchKernelGGL(qk_norm_rope_append_kernel<128>, dim3(units, tokens), dim3(64), 0, stream, P);
    else
        hipLaunchKernelGGL(qk_norm_rope_append_kernel<0>, dim3(units, tokens), dim3(64), 0, stream, P);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

Paged paged_of(const SimplerHipPaDecodeArgs *a, unsigned *error_flag, unsigned bad_length) {
    Paged G{};
    G.block_table = a->block_table;
    G.context_lens = a->context_lens;
    G.error_flag = error_flag;
    G.bad_length = bad_length;
    G.q_len = a->q_len;
    G.max_blocks = a->max_blocks_per_seq;
    return G;
}

}  // namespace
}  // namespace simpler_hip_kv

namespace simpler_hip {

using namespace simpler_hip_kv;

int launch_paged_append(const SimplerHipPaDecodeArgs *a, const void *key_new, const void *value_new,
                        unsigned *error_flag, unsigned bad_length, void *stream) {
    const int tokens = a->batch * a->q_len;
    if (tokens == 0) return SIMPLER_HIP_OK;
    AppendParams P{};
    P.key = (const uint16_t *)key_new;
    P.value = (const uint16_t *)value_new;
    P.kc = (uint16_t *)a->key_cache;
    P.vc = (uint16_t *)a->value_cache;
    P.key_ts = (int64_t)a->num_kv_heads * a->head_dim_k;
    P.key_hs = a->head_dim_k;
    P.val_ts = (int64_t)a->num_kv_heads * a->head_dim_v;
    P.val_hs = a->head_dim_v;
    P.k_bs = a->k_block_stride;
    P.k_ts = a->k_token_stride;
    P.k_hs = a->k_head_stride;
    P.v_bs = a->v_block_stride;
    P.v_ts = a->v_token_stride;
    P.v_hs = a->v_head_stride;
    P.num_tokens = tokens;
    P.hkv = a->num_kv_heads;
    P.dk = a->head_dim_k;
    P.dv = a->head_dim_v;
    P.block_size = a->block_size;
    P.num_blocks = a->num_blocks;
    P.pg = paged_of(a, error_flag, bad_length);
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)tokens), dim3(kThreads), 0, (hipStream_t)stream, P);
    return hipGetLastError() == hipSuccess ? SIMPLER_HIP_OK : SIMPLER_HIP_ERR_LAUNCH;
}

int launch_paged_prelude(const SimplerHipPaDecodeArgs *a, const SimplerHipDecodePreludeArgs *pre, void *q_out,
                         unsigned *error_flag, unsigned bad_length, void *stream) {
    const int tokens = a->batch * a->q_len;
    if (tokens == 0) return SIMPLER_HIP_OK;
    if (tokens > 65535) return SIMPLER_HIP_ERR_UNSUPPORTED;  // one grid row per token
    PreludeParams P{};
    P.q_proj = pre->q_proj;
    P.k_proj = pre->k_proj;
    P.v_proj = pre->v_proj;
    P.inv_rms = pre->inv_rms;
    P.q_w = pre->q_norm_weight;
    P.k_w = pre->k_norm_weight;
    P.cos = pre->rope_cos;
    P.sin = pre->rope_sin;
    P.q_out = (uint16_t *)q_out;
    P.kc = (uint16_t *)a->key_cache;
    P.vc = (uint16_t *)a->value_cache;
    P.k_bs = a->k_block_stride;
    P.k_ts = a->k_token_stride;
    P.k_hs = a->k_head_stride;
    P.v_bs = a->v_block_stride;
    P.v_ts = a->v_token_stride;
    P.v_hs = a->v_head_stride;
    P.batch = tokens;
    P.hq = a->num_heads;
    P.hkv = a->num_kv_heads;
    P.d = a->head_dim_k;
    P.block_size = a->block_size;
    P.num_blocks = a->num_blocks;
    P.max_pos = pre->max_position;
    P.eps = pre->eps;
    P.pg = paged_of(a, error_flag, bad_length);
    launch_prelude_kernel(P, (unsigned)(a->num_heads + 2 * a->num_kv_heads), (unsigned)tokens, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? SIMPLER_HIP_OK : SIMPLER_HIP_ERR_LAUNCH;
}

}  // namespace simpler_hip

using namespace simpler_hip_kv;

extern "C" int simpler_hip_kv_append(const SimplerHipKvAppendArgs *a, void *stream) {
    if (!a || !a->key || !a->slot_mapping || !a->key_cache) return SIMPLER_HIP_ERR_INVALID;
    if ((a->value == nullptr) != (a->value_cache == nullptr)) return SIMPLER_HIP_ERR_INVALID;
    if (a->num_tokens < 0 || a->num_kv_heads < 1 || a->block_size < 1 || a->num_blocks < 1)
        return SIMPLER_HIP_ERR_INVALID;
    if (a->head_dim_k < 8 || a->head_dim_k % 8 || a->head_dim_k > kMaxHeadDim) return SIMPLER_HIP_ERR_INVALID;
    if (a->value && (a->head_dim_v < 8 || a->head_dim_v % 8 || a->head_dim_v > kMaxHeadDim))
        return SIMPLER_HIP_ERR_INVALID;
    const int64_t strides[10] = {a->key_token_stride, a->key_head_stride, a->k_block_stride, a->k_token_stride,
                                 a->k_head_stride,    a->value_token_stride, a->value_head_stride,
                                 a->v_block_stride,   a->v_token_stride,  a->v_head_stride};
    for (int i = 0; i < 10; ++i) {
        const bool is_v = i >= 5;
        if (is_v && !a->value) continue;
        if (strides[i] <= 0 || strides[i] % 8) return SIMPLER_HIP_ERR_INVALID;  // 16-byte rows
    }
    if (!aligned16(a->key) || !aligned16(a->key_cache) || (a->value && (!aligned16(a->value) ||
                                                                          !aligned16(a->value_cache))))
        return SIMPLER_HIP_ERR_INVALID;
    if (a->num_tokens == 0) return SIMPLER_HIP_OK;
    AppendParams P{};
    P.key = (const uint16_t *)a->key;
    P.value = (const uint16_t *)a->value;
    P.slot = a->slot_mapping;
    P.kc = (uint16_t *)a->key_cache;
    P.vc = (uint16_t *)a->value_cache;
    P.err = a->error_count;
    P.key_ts = a->key_token_stride;
    P.key_hs = a->key_head_stride;
    P.val_ts = a->value_token_stride;
    P.val_hs = a->value_head_stride;
    P.k_bs = a->k_block_stride;
    P.k_ts = a->k_token_stride;
    P.k_hs = a->k_head_stride;
    P.v_bs = a->v_block_stride;
    P.v_ts = a->v_token_stride;
    P.v_hs = a->v_head_stride;
    P.num_tokens = a->num_tokens;
    P.hkv = a->num_kv_heads;
    P.dk = a->head_dim_k;
    P.dv = a->head_dim_v;
    P.block_size = a->block_size;
    P.num_blocks = a->num_blocks;
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)a->num_tokens), dim3(kThreads), 0, (hipStream_t)stream, P);
    return hipGetLastError() == hipSuccess ? SIMPLER_HIP_OK : SIMPLER_HIP_ERR_LAUNCH;
}

extern "C" int simpler_hip_qk_norm_rope_append(const SimplerHipQkNormRopeAppendArgs *a, void *stream) {
    if (!a || !a->q_proj || !a->k_proj || !a->v_proj || !a->inv_rms || !a->q_norm_weight || !a->k_norm_weight ||
        !a->rope_cos || !a->rope_sin || !a->seq_lens || !a->slot_mapping || !a->q_out || !a->key_cache ||
        !a->value_cache)
        return SIMPLER_HIP_ERR_INVALID;
    if (a->batch < 0 || a->num_heads < 1 || a->num_kv_heads < 1 || a->block_size < 1 || a->num_blocks < 1 ||
        a->max_position < 1)
        return SIMPLER_HIP_ERR_INVALID;
    if (a->head_dim < 2 || a->head_dim % 2 || a->head_dim > kMaxHeadDim) return SIMPLER_HIP_ERR_INVALID;
    const int64_t strides[6] = {a->k_block_stride, a->k_token_stride, a->k_head_stride,
                                a->v_block_stride, a->v_token_stride, a->v_head_stride};
    for (int64_t s : strides)
        if (s <= 0) return SIMPLER_HIP_ERR_INVALID;
    if (!(a->eps >= 0.f)) return SIMPLER_HIP_ERR_INVALID;
    if (a->batch == 0) return SIMPLER_HIP_OK;
    PreludeParams P{};
    P.q_proj = a->q_proj;
    P.k_proj = a->k_proj;
    P.v_proj = a->v_proj;
    P.inv_rms = a->inv_rms;
    P.q_w = a->q_norm_weight;
    P.k_w = a->k_norm_weight;
    P.cos = a->rope_cos;
    P.sin = a->rope_sin;
    P.seq_lens = a->seq_lens;
    P.slot = a->slot_mapping;
    P.q_out = (uint16_t *)a->q_out;
    P.kc = (uint16_t *)a->key_cache;
    P.vc = (uint16_t *)a->value_cache;
    P.err = a->error_count;
    P.k_bs = a->k_block_stride;
    P.k_ts = a->k_token_stride;
    P.k_hs = a->k_head_stride;
    P.v_bs = a->v_block_stride;
    P.v_ts = a->v_token_stride;
    P.v_hs = a->v_head_stride;
    P.batch = a->batch;
    P.hq = a->num_heads;
    P.hkv = a->num_kv_heads;
    P.d = a->head_dim;
    P.block_size = a->block_size;
    P.num_blocks = a->num_blocks;
    P.max_pos = a->max_position;
    P.eps = a->eps;
    launch_prelude_kernel(P, (unsigned)(a->num_heads + 2 * a->num_kv_heads), (unsigned)a->batch,
                          (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? SIMPLER_HIP_OK : SIMPLER_HIP_ERR_LAUNCH;
}
