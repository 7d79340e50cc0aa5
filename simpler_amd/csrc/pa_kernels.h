// Fused split-K paged-attention decode for gfx950 (MI355X).
//
// Replaces the per-KV-block AICore task chain of simpler's paged attention
// (examples/a2a3/tensormap_and_ringbuffer/paged_attention/kernels/):
//   QK  aic/aic_qk_matmul.cpp:38-100        -> MFMA 16x16x32 bf16, S^T = K * Q^T
//   SF  aiv/aiv_softmax_prepare.cpp:96-131  -> in-register mask/scale/rowmax/exp,
//                                             P rounded to bf16 (RNE) before the
//                                             row sum and before PV
//   PV  aic/aic_pv_matmul.cpp:38-99         -> MFMA 16x16x16 bf16, O += P * V
//   UP  aiv/aiv_online_update.cpp:125-224   -> register-resident online merge
// plus the cross-split log-sum-exp merge of the reference's SplitKV path
// (tests/st/a2a3/tensormap_and_ringbuffer/spmd_paged_attention_highperf/
//  kernels/kernel/pa_kernel.cce:1634-1773), done by a second kernel.
//
// Numerics follow the reference golden (simpler_setup/goldens/paged_attention.py
// :145-187) block for block: the softmax max is taken per KV block, p is rounded
// to bf16 relative to that block max, l sums the rounded p, and blocks merge
// with m' = max(m, m_blk). The accumulator is kept in the frame of the latest
// block max ("block frame": A = O * e^{m - f}), so the per-block merge
//   O' = e^{m-m'} O + e^{m_blk-m'} (P_blk V)
// becomes A' = e^{f - m_blk} A + P_blk V, which MFMA accumulates in place.
// A block whose max lies more than kFrameGap below the running max adds less
// than e^-kFrameGap relative and is skipped, which bounds A by e^kFrameGap * |O|.
//
// Work decomposition (stream-K): the work is the flattened list of
// (tile, KV block) pairs, tile = (batch, kv head, row tile), in that order
// (optionally as one list per tile of a batch; see lane_tiles).
// A row is one (query token, head in the GQA group) pair; 16 rows per tile
// (MFMA N). The main kernel launches one worker (a wavefront; a wavefront
// running two row tiles of a kv head; or sibling wavefronts for several row
// tiles) per slot of the GPU (CUs x workers per CU at this kernel's
// occupancy) and gives each an equal contiguous slice of that
// list, computed on the device from context_lens, so ragged lengths cost no
// imbalance and no tail. A tile that
// lies inside one slice is finished (normalised and stored) by that wave; a
// tile cut by slice boundaries leaves one partial (O, m, l) per piece, and a
// second small kernel merges those by log-sum-exp. The kernel boundary orders
// the partial writes before the merge; no device-scope fences are used.
//
// Lane (qd = lane/16, pc = lane%16):
//   QK   A operand = K token pc of the tile, dims 32kk+8qd..+7 (one 16-B load,
//                    or one 16-B LDS read when K is staged through LDS)
//        B operand = Q row pc, same dims
//        C         = S[row pc][tokens 4qd..4qd+3]   (S^T tile)
//   PV   A operand = P[row pc][tokens 4qd..4qd+3]  == the QK C layout (no shuffle)
//        B operand = V[tokens 4qd..4qd+3][dim 8pc+jj], built from four 16-B row
//                    loads by an in-register 4x8 bf16 transpose
//        C         = O[rows 4qd..4qd+3][dim 8pc+jj]
// Within a segment, V of block i is issued first and K of block i+1 as soon
// as K of block i is consumed (after QK(i), or once K(i) is staged in LDS), so
// both streams are in flight during the math.
//
// Fused KV append (APPEND): the q_len new tokens of each sequence, given
// beside the caches, are its last positions. The blocks holding them run
// after the pipelined loop (unpipelined_blocks), where the new rows replace
// the cache's rows in registers and row tile 0's wave writes them into the
// caches (simpler_setup/goldens/qwen3_14b_decode.py:106-115,261-269 is the
// append this replaces).

#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "simpler_hip/pa_decode.h"

namespace simpler_hip {
namespace pa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
#define LDS_AS __attribute__((address_space(3)))

constexpr float kNegClamp = -1e30f;  // goldens/paged_attention.py:160 clamp
constexpr float kFrameGap = 40.f;
constexpr int kWorkersPerCu = 2;       // default worker workgroups per compute unit (half-line K reads)
constexpr int kWorkersPerSimdCu = 4;   // one worker per SIMD: full-row K reads (see make_plan)
constexpr int kWorkersThreePerCu = 3;  // fp8 caches and two-tile waves: three single-wave workers per CU
constexpr int kMaxWavesPerWorker = 4;  // row tiles per worker workgroup (256 threads)

struct KernelParams {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    const int32_t *block_table;
    const int32_t *context_lens;
    void *out;
    float *part_o;   // [workers][2 slots][16 rows][DV]
    float *part_ml;  // [workers][2 slots][m[16], l[16]]
    unsigned *error_flag;
    const char *zeros;  // 256 bytes of the workspace that stay zero (LDS fill source)
    const char *zero_page;  // zero bytes standing in for the 16-token tiles past a context's end, or null
    const float *k_scale;  // fp8 caches: [num_blocks][kv_heads] dequantisation scales
    const float *v_scale;
    int64_t k_block_stride, k_token_stride, k_head_stride;
    int64_t v_block_stride, v_token_stride, v_head_stride;
    int32_t batch, q_len, num_heads, kv_heads, group, rows, row_tiles;
    int32_t tiles_per_worker;  // row tiles a worker workgroup runs side by side (one wave each)
    int32_t row_groups;        // ceil(row_tiles / tiles_per_worker): work-list tiles per kv head
    int32_t block_size, max_blocks, num_pool_blocks;
    int32_t workers;
    int32_t lanes;  // independent work lists; list u holds tiles [u, u+1) * (tiles per batch / lanes) of each batch
    float scale;
    int32_t causal;
    unsigned *err_mirror;  // host-visible copy of *error_flag written by the merge kernel, or null
    // Work units charged at the start of each work-list tile ahead of its
    // blocks (0: a slice's work is its block count). A slice that starts
    // further tiles pays for each one's set-up (query rows, first fill,
    // partial or output stores) in blocks it does not get.
    int32_t seg_cost;
    // fused KV append: the q_len new tokens of each sequence (its positions
    // len-q_len .. len-1), [batch, q_len, kv_heads, Dk] and [.., Dv]; v_new is
    // null for MLA (V is a prefix of K). Null when not appending.
    const uint16_t *k_new;
    const uint16_t *v_new;
};

__device__ __forceinline__ u32x4_t ld16(const uint16_t *p) { return *reinterpret_cast<const u32x4_t *>(p); }

// V rows are read as whole 128-byte lines exactly once: non-temporal loads
// keep them from displacing useful lines (measured ~11% more read bandwidth on
// MI355X than plain loads). K is read as 64-byte halves of a line by two
// consecutive instructions, so K uses plain loads, which let the L1 merge the
// two halves into one line request (non-temporal K measured 5-10% slower).
__device__ __forceinline__ u32x4_t stream_ld16(const char *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
}

__device__ __forceinline__ u32x4_t lds_ld16(const char *base, uint32_t off) {
    return *reinterpret_cast<const LDS_AS u32x4_t *>((const LDS_AS char *)base + off);
}

__device__ __forceinline__ void lds_st16(char *base, uint32_t off, u32x4_t v) {
    *reinterpret_cast<LDS_AS u32x4_t *>((LDS_AS char *)base + off) = v;
}

// Orders one wave's LDS writes before its later reads of other lanes' data
// (and those reads before later writes). The LDS executes a wave's
// instructions in order, so this only has to stop the compiler from moving
// LDS accesses across it; it emits no instruction.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ unsigned pack_bf16x2(float a, float b) {
    // fp32 -> bf16 round-to-nearest-even (gfx950: v_cvt_pk_bf16_f32)
    const bf16x2_t h = __builtin_convertvector((f32x2_t){a, b}, bf16x2_t);
    return __builtin_bit_cast(unsigned, h);
}

// The 16-bit element type of the query and the caches: its MFMA forms and
// the rounding of p to it (the golden rounds p to the input dtype before the
// row sum and PV, goldens/paged_attention.py:168; the reference's GQA cases
// are fp16, tests/st/.../spmd_paged_attention_highperf/
// test_spmd_paged_attention_highperf.py:170-232).
template <typename ET>
struct Elem;

template <>
struct Elem<__bf16> {
    static constexpr unsigned kOnePair = 0x3f803f80u;  // two bf16 1.0
    // 16x16x32: 8 elements per lane of each operand
    static __device__ __forceinline__ f32x4_t mma32(u32x4_t a, u32x4_t b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       c, 0, 0, 0);
    }
    // 16x16x16: 4 elements per lane of each operand
    static __device__ __forceinline__ f32x4_t mma16(u32x2_t a, u32x2_t b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, a), __builtin_bit_cast(i16x4_t, b),
                                                         c, 0, 0, 0);
    }
    static __device__ __forceinline__ unsigned pack2(float a, float b) { return pack_bf16x2(a, b); }
};

template <>
struct Elem<_Float16> {
    static constexpr unsigned kOnePair = 0x3c003c00u;  // two fp16 1.0
    static __device__ __forceinline__ f32x4_t mma32(u32x4_t a, u32x4_t b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                      0, 0, 0);
    }
    static __device__ __forceinline__ f32x4_t mma16(u32x2_t a, u32x2_t b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a), __builtin_bit_cast(f16x4_t, b), c,
                                                     0, 0, 0);
    }
    // fp32 -> fp16 round-to-nearest-even (gfx950: v_cvt_pk_f16_f32)
    static __device__ __forceinline__ unsigned pack2(float a, float b) {
        return __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
    }
};

// P x V (and P x ones) over two 16-token tiles in one 16x16x32 MFMA: lane
// (pc, qd) holds k-steps 8qd .. 8qd+7 of its A and B operands; the first four
// are tile 0's tokens 4qd .. 4qd+3 (its 16x16x16 operands a0, b0), the last
// four tile 1's (a1, b1), the same order in A and B, so the product sums
// over all 32 tokens: one instruction where the 16x16x16 form takes two.
// kTilePairs: where it is used. The single-tile waves (fp8 56.9 against 57.4
// us per main launch in same-box pairs; cfg2, cfg3 and cfg1 unchanged); the
// two-tile wave measured slower with it (the verify shape 138.3 against
// 134.0) and keeps one 16x16x16 MFMA per tile.
template <int NT, int RTW>
constexpr bool kTilePairs = NT % 2 == 0 && RTW == 1;

template <typename ET>
__device__ __forceinline__ f32x4_t mma_tile_pair(const u32x2_t a0, const u32x2_t a1, const u32x2_t b0,
                                                 const u32x2_t b1, const f32x4_t c) {
    return Elem<ET>::mma32((u32x4_t){a0[0], a0[1], a1[0], a1[1]}, (u32x4_t){b0[0], b0[1], b1[0], b1[1]}, c);
}

// Four E4M3FN bytes -> four bf16 (two words); exact (every E4M3FN value is a
// bf16 value). gfx950 v_cvt_scalef32_pk_bf16_fp8 with scale 1.
__device__ __forceinline__ u32x2_t fp8x4_to_bf16x4(unsigned w) {
    const bf16x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    const bf16x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    return (u32x2_t){__builtin_bit_cast(unsigned, lo), __builtin_bit_cast(unsigned, hi)};
}

// Eight E4M3FN bytes (two words) -> eight bf16 (one 16-byte MFMA operand).
__device__ __forceinline__ u32x4_t fp8x8_to_bf16x8(unsigned w0, unsigned w1) {
    const u32x2_t a = fp8x4_to_bf16x4(w0), b = fp8x4_to_bf16x4(w1);
    return (u32x4_t){a[0], a[1], b[0], b[1]};
}


template <typename OutT>
struct OutStore;

template <>
struct OutStore<float> {
    // 8 consecutive values
    __device__ static void store8(void *base, int64_t off, const float (&v)[8]) {
        float *p = reinterpret_cast<float *>(base) + off;
        *reinterpret_cast<f32x4_t *>(p) = (f32x4_t){v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4_t *>(p + 4) = (f32x4_t){v[4], v[5], v[6], v[7]};
    }
    __device__ static void store4(void *base, int64_t off, f32x4_t v) {
        *reinterpret_cast<f32x4_t *>(reinterpret_cast<float *>(base) + off) = v;
    }
};

template <>
struct OutStore<_Float16> {
    __device__ static void store8(void *base, int64_t off, const float (&v)[8]) {
        uint16_t *p = reinterpret_cast<uint16_t *>(base) + off;
        *reinterpret_cast<u32x4_t *>(p) =
            (u32x4_t){Elem<_Float16>::pack2(v[0], v[1]), Elem<_Float16>::pack2(v[2], v[3]),
                      Elem<_Float16>::pack2(v[4], v[5]), Elem<_Float16>::pack2(v[6], v[7])};
    }
    __device__ static void store4(void *base, int64_t off, f32x4_t v) {
        uint16_t *p = reinterpret_cast<uint16_t *>(base) + off;
        *reinterpret_cast<u32x2_t *>(p) = (u32x2_t){Elem<_Float16>::pack2(v[0], v[1]), Elem<_Float16>::pack2(v[2], v[3])};
    }
};

template <>
struct OutStore<__bf16> {
    __device__ static void store8(void *base, int64_t off, const float (&v)[8]) {
        uint16_t *p = reinterpret_cast<uint16_t *>(base) + off;
        *reinterpret_cast<u32x4_t *>(p) = (u32x4_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                    pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
    }
    __device__ static void store4(void *base, int64_t off, f32x4_t v) {
        uint16_t *p = reinterpret_cast<uint16_t *>(base) + off;
        *reinterpret_cast<u32x2_t *>(p) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
};

// ---------------------------------------------------------------------------
// Work partition shared by both kernels
// ---------------------------------------------------------------------------

// Context length of sequence b, clamped to what its block-table row can hold.
__device__ __forceinline__ int ctx_of(const KernelParams &P, int b) {
    return min(max(P.context_lens[b], 0), P.max_blocks * P.block_size);
}

__device__ __forceinline__ int blocks_of(const KernelParams &P, int b) {
    return (ctx_of(P, b) + P.block_size - 1) / P.block_size;
}

// Error word bits (workspace offset 0), read back by simpler_hip_pa_decode_check.
constexpr unsigned kErrBadBlock = 1u;   // a block_table entry outside the pool (that block is skipped)
constexpr unsigned kErrBadLength = 2u;  // a context_lens entry the kernels had to clamp

constexpr int kScanGroup = 8;

// The raw lengths of sequences base0 + 64 k + lane (k < kScanGroup), from
// clamped indices and all loaded before any is used: the empty asm needs all
// eight, so the compiler can neither sink a load into the past-the-batch
// branch that uses it nor wait for each in turn (one memory round trip, not
// eight).
__device__ __forceinline__ void load_lengths(const KernelParams &P, const int base0, int (&lens)[kScanGroup]) {
    static_assert(kScanGroup == 8, "the load fence below names each length");
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < kScanGroup; ++k) {
        const int b = base0 + 64 * k + lane;
        lens[k] = P.context_lens[b < P.batch ? b : 0];
    }
    asm volatile("" : "+v"(lens[0]), "+v"(lens[1]), "+v"(lens[2]), "+v"(lens[3]), "+v"(lens[4]), "+v"(lens[5]),
                 "+v"(lens[6]), "+v"(lens[7]));
}

// One wave of the grid (wave 0 of workgroup 0) checks every raw length: below
// 0, above what the block-table row holds, or (causal) shorter than the query.
// With a fused append, a length below q_len cannot hold the new tokens. The
// kernels run such a sequence with its length clamped by ctx_of; the flag
// turns that into an error for the caller, as the host-side table check does.
__device__ __forceinline__ void flag_bad_lengths(const KernelParams &P) {
    if (blockIdx.x != 0 || threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const int64_t cap = (int64_t)P.max_blocks * P.block_size;
    const int lo = (P.causal || P.k_new) ? P.q_len : 0;  // an appended context holds its new tokens
    bool bad = false;
    if (P.batch <= 64) {
        const int len = lane < P.batch ? P.context_lens[lane] : 0;
        bad = lane < P.batch && (len < lo || (int64_t)len > cap);
    }
    for (int base0 = 0; P.batch > 64 && base0 < P.batch; base0 += 64 * kScanGroup) {
        int lens[kScanGroup];
        load_lengths(P, base0, lens);
#pragma unroll
        for (int k = 0; k < kScanGroup; ++k)
            bad |= base0 + 64 * k + lane < P.batch && (lens[k] < lo || (int64_t)lens[k] > cap);
    }
    if (__ballot(bad) && lane == 0) atomicOr(P.error_flag, kErrBadLength);
}

// Work lists: the (tile, KV block) pairs of all batches form P.lanes lists of
// equal length. List u holds, per batch, the tiles u*lt .. u*lt+lt-1 (lt =
// tiles per batch / lanes), batch-major, then tile, then block; its
// P.workers / lanes workers (ids u, u + lanes, u + 2*lanes, ...) take equal
// contiguous slices of it. With lanes = tiles per batch, the workers of every
// kv head get the same block ranges, so neighbouring workers read the
// different heads of the same token rows at about the same time (the caches
// interleave heads within a row).
__device__ __forceinline__ int lane_tiles(const KernelParams &P) { return P.kv_heads * P.row_groups / P.lanes; }

// Which tiles a list takes rotates with the batch: list u runs tile group
// (u + b) mod lanes of batch b. Every list (and so every worker) then meets
// every kv head, whose K/V streams run at different speeds depending on how
// their rows map onto memory channels, instead of one list per head setting
// the kernel's end. Neighbouring lists still read the heads of the same token
// rows together.
__device__ __forceinline__ int list_tile0(const KernelParams &P, int list, int b) {
    return ((list + b) % P.lanes) * lane_tiles(P);
}
// The list that ran tile group g of batch b.
__device__ __forceinline__ int list_of_tile(const KernelParams &P, int g, int b) {
    return ((g - b) % P.lanes + P.lanes) % P.lanes;
}

// Work of sequence b (raw length len) for the scans below: (blocks +
// seg_cost) * tiles per batch, 0 for an empty context or past the batch.
__device__ __forceinline__ int work_of(const KernelParams &P, const int b, const int len, const int tpb) {
    const int ctx = min(max(len, 0), P.max_blocks * P.block_size);
    const int nbb = b < P.batch ? (ctx + P.block_size - 1) / P.block_size : 0;
    return nbb > 0 ? (nbb + P.seg_cost) * tpb : 0;
}

// Inclusive wave scan of x by DPP lane moves (no LDS round trips, which
// __shfl_up takes): row_shr 1, 2, 4, 8 within each 16-lane row (lanes past a
// row's start read 0), then row_bcast:15 adds the last lane of rows 0 and 2
// to rows 1 and 3, and row_bcast:31 lane 31 to rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
    return x;
}

// Wave-level scan over the batch for one list. Work of batch b = (blocks_of(b)
// + seg_cost) * lane_tiles, or 0 for an empty context. Returns the total
// work; if `want_b` >= 0, *prefix_of_want = work before batch want_b and
// *ctx_of_want = its clamped length (ctx_of); if `pos` >= 0 (and < total),
// *b_of_pos / *prefix_of_pos / *ctx_of_pos = the batch whose work range
// contains pos, the work before it and its clamped length. All results are
// wave-uniform. Each group of up to 64 * kScanGroup sequences costs one memory
// round trip.
__device__ inline int scan_work(const KernelParams &P, int want_b, int *prefix_of_want, int *ctx_of_want, int pos,
                                int *b_of_pos, int *prefix_of_pos, int *ctx_of_pos) {
    const int lane = threadIdx.x & 63;
    const int tpb = lane_tiles(P);
    const int cap = P.max_blocks * P.block_size;
    int carry = 0;
    for (int base0 = 0; base0 < P.batch; base0 += 64 * kScanGroup) {
        int lens[kScanGroup];
        load_lengths(P, base0, lens);
#pragma unroll
        for (int k = 0; k < kScanGroup; ++k) {
            const int base = base0 + 64 * k;
            if (base >= P.batch) break;  // wave-uniform
            const int cnt = work_of(P, base + lane, lens[k], tpb);
            const int incl = wave_incl_scan(cnt);
            const int excl = carry + incl - cnt;
            const int ctx = min(max(lens[k], 0), cap);
            if (want_b >= base && want_b < base + 64) {
                *prefix_of_want = __shfl(excl, want_b - base, 64);
                *ctx_of_want = __shfl(ctx, want_b - base, 64);
            }
            if (pos >= 0) {
                const unsigned long long hit = __ballot(cnt > 0 && pos >= excl && pos < excl + cnt);
                if (hit) {
                    const int src = __ffsll((long long)hit) - 1;
                    *b_of_pos = base + src;
                    *prefix_of_pos = __shfl(excl, src, 64);
                    *ctx_of_pos = __shfl(ctx, src, 64);
                }
            }
            carry += __shfl(incl, 63, 64);
        }
    }
    return carry;
}

// Slice c of a list (the list's c-th worker): [*start, *end) of its work
// units, and the batch holding *start with the work before it and its clamped
// length. Up to 64 * kScanGroup sequences take one memory round trip: their
// lengths stay in registers between the total and the search for the start
// (up to 64, one per lane).
__device__ inline int locate_slice(const KernelParams &P, int c, int *start, int *end, int *b_of_start,
                                   int *prefix_of_start, int *ctx_of_start) {
    const int lane = threadIdx.x & 63;
    const int per_list = max(P.workers / P.lanes, 1);
    if (P.batch > 64 * kScanGroup) {
        const int total = scan_work(P, -1, nullptr, nullptr, -1, nullptr, nullptr, nullptr);
        const int chunk = (total + per_list - 1) / per_list;
        *start = c * chunk;
        *end = min(*start + chunk, total);
        if (*start < *end) scan_work(P, -1, nullptr, nullptr, *start, b_of_start, prefix_of_start, ctx_of_start);
        return total;
    }
    const int tpb = lane_tiles(P);
    const int cap = P.max_blocks * P.block_size;
    if (P.batch <= 64) {  // one length per lane
        const int ctxl = lane < P.batch ? min(max(P.context_lens[lane], 0), cap) : 0;
        const int nbl = (ctxl + P.block_size - 1) / P.block_size;
        const int cnt = nbl > 0 ? (nbl + P.seg_cost) * tpb : 0;
        const int incl = wave_incl_scan(cnt);
        const int total = __shfl(incl, 63, 64);
        const int chunk = (total + per_list - 1) / per_list;
        *start = c * chunk;
        *end = min(*start + chunk, total);
        const int excl = incl - cnt;
        const unsigned long long hit = __ballot(cnt > 0 && *start >= excl && *start < excl + cnt);
        if (hit) {
            const int src = __ffsll((long long)hit) - 1;
            *b_of_start = src;
            *prefix_of_start = __shfl(excl, src, 64);
            *ctx_of_start = __shfl(ctxl, src, 64);
        }
        return total;
    }
    int lens[kScanGroup], cnts[kScanGroup], excl[kScanGroup];
    load_lengths(P, 0, lens);
    int carry = 0;
#pragma unroll
    for (int k = 0; k < kScanGroup; ++k) {
        cnts[k] = work_of(P, 64 * k + lane, lens[k], tpb);  // 0 past the batch
        excl[k] = carry;
        if (64 * k >= P.batch) continue;  // wave-uniform
        const int incl = wave_incl_scan(cnts[k]);
        excl[k] = carry + incl - cnts[k];
        carry += __shfl(incl, 63, 64);
    }
    const int total = carry;
    const int chunk = (total + per_list - 1) / per_list;
    *start = c * chunk;
    *end = min(*start + chunk, total);
#pragma unroll
    for (int k = 0; k < kScanGroup; ++k) {
        const unsigned long long hit = __ballot(cnts[k] > 0 && *start >= excl[k] && *start < excl[k] + cnts[k]);
        if (hit) {
            const int src = __ffsll((long long)hit) - 1;
            *b_of_start = 64 * k + src;
            *prefix_of_start = __shfl(excl[k], src, 64);
            *ctx_of_start = __shfl(min(max(lens[k], 0), cap), src, 64);
        }
    }
    return total;
}

// Output element offset of (row r of kv head kvh, dim 0).
__device__ __forceinline__ int64_t out_row_offset(const KernelParams &P, int b, int kvh, int r, int dv) {
    const int i = r / P.group, hh = r - i * P.group;
    return ((int64_t)(b * P.q_len + i) * P.num_heads + kvh * P.group + hh) * dv;
}

// ---------------------------------------------------------------------------
// One segment: KV blocks [blk_begin, blk_end) of tile (b, kvh, rt)
// ---------------------------------------------------------------------------

// End of a segment (rows of row tile rt of (b, kvh), blocks [blk_begin,
// blk_end)): O = e^{f-m} A and l = e^{f-m} L in the frame of the running max m
// (A in units of vs_frame for fp8 V), then either the final output (the
// segment covers the whole tile) or the tile piece (O relative to m, m, l)
// for the merge kernel. Lane (qd, pc) holds A's rows 4qd+e and the state of
// row pc.
template <int DV, typename OutT>
__device__ __forceinline__ void finish_segment(const KernelParams &P, const int b, const int kvh, const int rt,
                                               const int nblk, const int blk_begin, const int blk_end,
                                               float *const part_o, float *const part_ml,
                                               const f32x4_t (&acc)[(DV + 127) / 128][8], const f32x4_t lacc,
                                               const float m_run, const float f_run, const float vs_frame) {
    constexpr int DVS = (DV + 127) / 128;
    const int lane = threadIdx.x & 63;
    const int qd = lane >> 4;
    const int pc = lane & 15;
    const int rows_here = min(16, P.rows - rt * 16);
    const float oscl = __expf(f_run - m_run);  // row pc's
    const float osc = oscl * vs_frame;
    float l_e[4], o_e[4];  // rows 4qd+e
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        l_e[e] = lacc[e] * __shfl(oscl, 4 * qd + e, 64);
        o_e[e] = __shfl(osc, 4 * qd + e, 64);
    }
    // row pc's l: element pc % 4 of the lanes of group pc / 4
    float l_tot;
    {
        float lr[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) lr[e] = __shfl(l_e[e], 16 * (pc >> 2) + pc, 64);
        const int ep = pc & 3;
        l_tot = ep == 0 ? lr[0] : ep == 1 ? lr[1] : ep == 2 ? lr[2] : lr[3];
    }

    if (blk_begin == 0 && blk_end == nblk) {  // the whole tile: final output
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = 4 * qd + e;
            if (row >= rows_here) continue;
            const int64_t off = out_row_offset(P, b, kvh, rt * 16 + row, DV);
#pragma unroll
            for (int ds = 0; ds < DVS; ++ds) {
                if (!(DV % 128 == 0 || 128 * ds + 8 * pc < DV)) continue;
                float v[8];
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) v[jj] = l_e[e] > 0.f ? (o_e[e] * acc[ds][jj][e]) / l_e[e] : 0.f;
                OutStore<OutT>::store8(P.out, off + 128 * ds + 8 * pc, v);
            }
        }
        return;
    }

    // ---- a piece of the tile: partial (O relative to m, plus m and l) ----
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int row = 4 * qd + e;
        if (row >= rows_here) continue;
#pragma unroll
        for (int ds = 0; ds < DVS; ++ds) {
            if (!(DV % 128 == 0 || 128 * ds + 8 * pc < DV)) continue;
            float *dst = part_o + row * DV + 128 * ds + 8 * pc;
            *reinterpret_cast<f32x4_t *>(dst) =
                (f32x4_t){acc[ds][0][e], acc[ds][1][e], acc[ds][2][e], acc[ds][3][e]} * o_e[e];
            *reinterpret_cast<f32x4_t *>(dst + 4) =
                (f32x4_t){acc[ds][4][e], acc[ds][5][e], acc[ds][6][e], acc[ds][7][e]} * o_e[e];
        }
    }
    if (qd == 0) {
        part_ml[pc] = m_run;
        part_ml[16 + pc] = l_tot;
    }
}

// Fused KV append. The q_len (<= 16) new tokens of sequence b are its
// positions len-q_len .. len-1 (len = context_lens[b]; ctx = len once it is
// in range). They are consecutive, so each residue of a
// position mod 16 belongs to one new token at most, and a lane, whose K and V
// operands always hold the same residues (register K: token pc of every
// 16-token tile; V and row-staged K: tokens 4qd+e), needs the rows of at most
// one new token per residue it holds, loaded once per segment. Every wave
// that reads a block holding new tokens uses these rows in place of the
// cache's (so what the cache holds there during the launch never matters),
// and the wave of row tile 0 writes them into the cache.
__device__ __forceinline__ int new_token_at(const int new0, const int ctx, const int r) {
    const int p = new0 + ((r - new0) & 15);
    return (p >= 0 && p < ctx) ? p : -1;
}
// 16-token tile of block blk that holds position p, or -1
template <int BS>
__device__ __forceinline__ int tile_of(const int p, const int blk) {
    const int o = p - blk * BS;
    return (p >= 0 && (unsigned)o < (unsigned)BS) ? (o >> 4) : -1;
}

// ---------------------------------------------------------------------------
// KV blocks without cross-block prefetch, continuing a segment's state (A,
// its row sums, m, f). Two users:
//  * blocks whose K or V does not fit the registers as a whole (block_size x
//    head_dim above 16384 elements, e.g. 128 tokens x 256 dims): the block's
//    K and V are loaded in groups of GT 16-token tiles; QK runs over every
//    tile of the block before the softmax, whose max is the whole block's
//    (as the golden's), then PV group by group;
//  * the fused append's blocks that hold new tokens (APPEND), at the end of
//    a segment: the new rows are loaded here and replace the cache's rows in
//    registers (see new_token_at), so the pipelined loop before them carries
//    no extra registers.
// Same lane layouts and arithmetic as run_segment's register path, so a
// block gives the same bits either way. Blocks [lo, hi) of the segment that
// starts at blk_begin.
// ---------------------------------------------------------------------------

// RTW row tiles rt, rt+1, .. of one wave (each K and V operand feeds every
// tile's MFMAs); min_rowlen is the first tile's (the shortest).
template <int BS, int DK, int DV, typename ET, bool APPEND, int RTW = 1>
__device__ __forceinline__ void unpipelined_blocks(const KernelParams &P, const int b, const int kvh, const int rt,
                                                   const int ctx, const int blk_begin, const int lo, const int hi,
                                                   const u32x4_t (&qv)[RTW][(DK + 31) / 32], const int (&rowlen)[RTW],
                                                   const int min_rowlen, f32x4_t (&acc)[RTW][(DV + 127) / 128][8],
                                                   f32x4_t (&lacc)[RTW], float (&m_run)[RTW], float (&f_run)[RTW]) {
    constexpr int NT = BS / 16;            // 16-token tiles per KV block
    constexpr int KS = (DK + 31) / 32;     // 32-dim k-steps of QK
    constexpr int DVS = (DV + 127) / 128;  // 128-dim column sets of PV
    // tiles per load group: at most 128 / RTW registers of K (KS x 4 per tile)
    // and 128 of V (DVS x 16 per tile)
    constexpr int GK = 32 / KS / RTW > 0 ? 32 / KS / RTW : 1;
    constexpr int GV = 8 / DVS > 0 ? 8 / DVS : 1;
    constexpr int GT0 = GK < GV ? GK : GV;
    constexpr int GT = GT0 < NT ? GT0 : NT;
    static_assert(NT % GT == 0, "load groups divide the block");
    const int lane = threadIdx.x & 63;
    const int qd = lane >> 4;
    const int pc = lane & 15;
    const __attribute__((address_space(4))) int32_t *bt_row =
        (const __attribute__((address_space(4))) int32_t *)(P.block_table + (int64_t)b * P.max_blocks);
    const u32x2_t ones4 = (u32x2_t){Elem<ET>::kOnePair, Elem<ET>::kOnePair};
    constexpr float kLog2e = 1.4426950408889634f;

    const int64_t k_tok_b = P.k_token_stride * 2, v_tok_b = P.v_token_stride * 2;
    const uint32_t k_lane = (uint32_t)(pc * k_tok_b + 16 * qd);
    const uint32_t v_lane = (uint32_t)(4 * qd * v_tok_b + 16 * pc);
    const char *k_head = reinterpret_cast<const char *>(P.k) + (int64_t)kvh * P.k_head_stride * 2;
    const char *v_head = reinterpret_cast<const char *>(P.v) + (int64_t)kvh * P.v_head_stride * 2;
    auto tile_base = [&](const char *blk_base, int blk, int t, int64_t tok_b) -> const char * {
        const bool past = P.zero_page && 16 * t >= ctx - blk * BS;
        return past ? P.zero_page : blk_base + (int64_t)(16 * t) * tok_b;
    };

    // fused append: register-K rows of the new token at residue pc, V rows of
    // those at residues 4qd+e. The new tokens sit at the raw length's last
    // q_len positions; those at or past the clamped ctx are not in the table
    // and are dropped (new_token_at), as the routed append drops them.
    const int new0 = max(P.context_lens[b], 0) - P.q_len;
    int pk = -1, pe[4] = {-1, -1, -1, -1};
    u32x4_t knew[APPEND ? KS : 1], vnew[APPEND ? 4 : 1][DVS];
    if constexpr (APPEND) {
        const int64_t row0 = (int64_t)b * P.q_len - new0;  // k_new row of position p: row0 + p
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) knew[kk] = (u32x4_t){0u, 0u, 0u, 0u};
        pk = new_token_at(new0, ctx, pc);
        if (pk >= 0) {
            const uint16_t *kr = P.k_new + ((row0 + pk) * P.kv_heads + kvh) * DK;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
                if (DK % 32 == 0 || 32 * kk + 8 * qd < DK) knew[kk] = ld16(kr + 32 * kk + 8 * qd);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            pe[e] = new_token_at(new0, ctx, 4 * qd + e);
#pragma unroll
            for (int ds = 0; ds < DVS; ++ds) {
                vnew[e][ds] = (u32x4_t){0u, 0u, 0u, 0u};
                if (pe[e] >= 0 && (DV % 128 == 0 || 128 * ds + 8 * pc < DV))
                    vnew[e][ds] = ld16(P.v_new + ((row0 + pe[e]) * P.kv_heads + kvh) * DV + 128 * ds + 8 * pc);
            }
        }
    }

    bool any_bad = false;
    for (int blk = lo; blk < hi; ++blk) {
        const int raw = bt_row[blk];
        const bool bad = (unsigned)raw >= (unsigned)P.num_pool_blocks;
        any_bad |= bad;
        const int phys = bad ? 0 : raw;
        const char *kb = k_head + (int64_t)phys * P.k_block_stride * 2;
        const char *vb = v_head + (int64_t)phys * P.v_block_stride * 2;
        const bool first = (blk == blk_begin);
        const bool blk_new = APPEND && blk * BS + BS > new0;  // the block holds new tokens (wave-uniform)
        const int tk = APPEND && blk_new ? tile_of<BS>(pk, blk) : -1;

        // ---- QK over every tile of the block, GT tiles of K at a time ----
        f32x4_t s[RTW][NT];
#pragma unroll
        for (int g = 0; g < NT; g += GT) {
            u32x4_t kr[GT][KS];
#pragma unroll
            for (int t = 0; t < GT; ++t) {
                const char *kt = tile_base(kb, blk, g + t, k_tok_b);
#pragma unroll
                for (int kk = 0; kk < KS; ++kk)
                    kr[t][kk] = (DK % 32 == 0 || 32 * kk + 8 * qd < DK)
                                    ? *reinterpret_cast<const u32x4_t *>(kt + k_lane + 64 * kk)
                                    : (u32x4_t){0u, 0u, 0u, 0u};
            }
            if constexpr (APPEND) {
                if (blk_new) {
#pragma unroll
                    for (int t = 0; t < GT; ++t)
#pragma unroll
                        for (int kk = 0; kk < KS; ++kk)
                            if (g + t == tk) kr[t][kk] = knew[kk];
                }
            }
#pragma unroll
            for (int t = 0; t < GT; ++t)
#pragma unroll
                for (int r = 0; r < RTW; ++r) {
                    f32x4_t c = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kk = 0; kk < KS; ++kk) c = Elem<ET>::mma32(kr[t][kk], qv[r][kk], c);
                    s[r][g + t] = c;
                }
        }

        // ---- softmax prepare and the online-merge factor (as run_segment) ----
        const float scale = P.scale;
        const bool prescale = !(scale > 0.f);
        const float sc = prescale ? 1.f : scale;
        const int blk0 = blk * BS;
        const bool full = !bad && (blk0 + BS <= min_rowlen);
        u32x2_t pa[RTW][NT];
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
            if (prescale) {
#pragma unroll
                for (int t = 0; t < NT; ++t) s[r][t] *= scale;
            }
            const int rvalid = bad ? 0 : rowlen[r] - blk0;
            if (!full) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (16 * t + 4 * qd + e >= rvalid) s[r][t][e] = -INFINITY;
            }
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[r][t][e]);
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mb = fmaxf(mx * sc, kNegClamp);
            const float mnew = first ? mb : fmaxf(m_run[r], mb);
            const bool use = first || (mb >= mnew - kFrameGap);
            const float cf = first ? 0.f : (use ? __expf(f_run[r] - mb) : 1.f);
            const float mb2 = use ? mb * kLog2e : INFINITY;
            const float sc2 = sc * kLog2e;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float p[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r][t][e], sc2, -mb2));
                pa[r][t] = (u32x2_t){Elem<ET>::pack2(p[0], p[1]), Elem<ET>::pack2(p[2], p[3])};
            }
            m_run[r] = mnew;
            if (use) f_run[r] = mb;
            {
                f32x4_t cv;
#pragma unroll
                for (int e = 0; e < 4; ++e) cv[e] = __shfl(cf, 4 * qd + e, 64);
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) acc[r][ds][jj] *= cv;
                lacc[r] *= cv;
            }
            // (tile pairs as run_segment forms them: the same bits either way)
            if constexpr (kTilePairs<NT, RTW>) {
#pragma unroll
                for (int t = 0; t < NT; t += 2)
                    lacc[r] = mma_tile_pair<ET>(pa[r][t], pa[r][t + 1], ones4, ones4, lacc[r]);
            } else {
#pragma unroll
                for (int t = 0; t < NT; ++t) lacc[r] = Elem<ET>::mma16(pa[r][t], ones4, lacc[r]);
            }
        }

        // ---- PV, GT tiles of V at a time; V rows past the context (or of an
        // out-of-pool block) are zeroed ----
        const int vvalid = bad ? 0 : min(BS, ctx - blk0);
#pragma unroll
        for (int g = 0; g < NT; g += GT) {
            u32x4_t vr[GT][DVS][4];
#pragma unroll
            for (int t = 0; t < GT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const char *vt = tile_base(vb, blk, g + t, v_tok_b) + (int64_t)e * v_tok_b;
                    const bool zero = 16 * (g + t) + 4 * qd + e >= vvalid;
#pragma unroll
                    for (int ds = 0; ds < DVS; ++ds) {
                        u32x4_t x = (u32x4_t){0u, 0u, 0u, 0u};
                        if (DV % 128 == 0 || 128 * ds + 8 * pc < DV)
                            x = *reinterpret_cast<const u32x4_t *>(vt + v_lane + 256 * ds);
                        if constexpr (APPEND) {
                            if (blk_new && tile_of<BS>(pe[e], blk) == g + t) x = vnew[e][ds];
                        }
                        vr[t][ds][e] = zero ? (u32x4_t){0u, 0u, 0u, 0u} : x;
                    }
                }
            auto v_words = [&](const int t, const int ds, const int jj) -> u32x2_t {
                const int w = jj >> 1;
                constexpr unsigned kLoHalves = 0x05040100u, kHiHalves = 0x07060302u;
                const unsigned sel = (jj & 1) ? kHiHalves : kLoHalves;
                return (u32x2_t){__builtin_amdgcn_perm(vr[t][ds][1][w], vr[t][ds][0][w], sel),
                                 __builtin_amdgcn_perm(vr[t][ds][3][w], vr[t][ds][2][w], sel)};
            };
            static_assert(!kTilePairs<NT, RTW> || GT % 2 == 0, "load groups of whole tile pairs");
            constexpr int TP = kTilePairs<NT, RTW> ? 2 : 1;  // token tiles per PV MFMA, as in run_segment
#pragma unroll
            for (int t = 0; t < GT; t += TP)
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const u32x2_t b0 = v_words(t, ds, jj);
                        if constexpr (TP == 2) {
                            const u32x2_t b1 = v_words(t + 1, ds, jj);
#pragma unroll
                            for (int r = 0; r < RTW; ++r)
                                acc[r][ds][jj] =
                                    mma_tile_pair<ET>(pa[r][g + t], pa[r][g + t + 1], b0, b1, acc[r][ds][jj]);
                        } else {
#pragma unroll
                            for (int r = 0; r < RTW; ++r)
                                acc[r][ds][jj] = Elem<ET>::mma16(pa[r][g + t], b0, acc[r][ds][jj]);
                        }
                    }
        }
        // the new tokens of this block into the caches (row tile 0's wave)
        if constexpr (APPEND) {
            if (blk_new && rt == 0 && !bad) {
                char *kw = const_cast<char *>(kb), *vw = const_cast<char *>(vb);
                if (tk >= 0) {
#pragma unroll
                    for (int kk = 0; kk < KS; ++kk)
                        if (DK % 32 == 0 || 32 * kk + 8 * qd < DK)
                            *reinterpret_cast<u32x4_t *>(kw + (int64_t)(pk - blk0) * k_tok_b +
                                                         2 * (32 * kk + 8 * qd)) = knew[kk];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (tile_of<BS>(pe[e], blk) < 0) continue;
#pragma unroll
                    for (int ds = 0; ds < DVS; ++ds)
                        if (DV % 128 == 0 || 128 * ds + 8 * pc < DV)
                            *reinterpret_cast<u32x4_t *>(vw + (int64_t)(pe[e] - blk0) * v_tok_b +
                                                         2 * (128 * ds + 8 * pc)) = vnew[e][ds];
                }
            }
        }
    }
    if (any_bad && lane == 0) atomicOr(P.error_flag, kErrBadBlock);
}

// Query operand (row pc of row tile rt, dims 32kk+8qd..) and the row's visible
// length; 0 rows past the tile's valid rows.
template <int DK>
__device__ __forceinline__ void load_query(const KernelParams &P, const int b, const int kvh, const int rt,
                                           const int ctx, u32x4_t (&qv)[(DK + 31) / 32], int &rowlen) {
    constexpr int KS = (DK + 31) / 32;
    const int lane = threadIdx.x & 63;
    const int qd = lane >> 4, pc = lane & 15;
    rowlen = 0;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qv[kk] = (u32x4_t){0u, 0u, 0u, 0u};
    if (pc < min(16, P.rows - rt * 16)) {
        const int r = rt * 16 + pc;
        const int i = r / P.group, hh = r - i * P.group;
        const uint16_t *qrow = P.q + ((int64_t)(b * P.q_len + i) * P.num_heads + kvh * P.group + hh) * DK;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
            if (DK % 32 == 0 || 32 * kk + 8 * qd < DK) qv[kk] = ld16(qrow + 32 * kk + 8 * qd);
        rowlen = P.causal ? ctx - (P.q_len - 1 - i) : ctx;
    }
}

// A segment of blocks too large for the registers (see unpipelined_blocks).
template <int BS, int DK, int DV, typename OutT, typename ET, bool APPEND = false>
__device__ __forceinline__ void run_segment_big(const KernelParams &P, const int b, const int kvh, const int rt,
                                                const int ctx, const int nblk, const int blk_begin, const int blk_end,
                                                float *const part_o, float *const part_ml) {
    constexpr int KS = (DK + 31) / 32;
    constexpr int DVS = (DV + 127) / 128;
    u32x4_t qv[1][KS];
    int rowlen[1] = {0};
    load_query<DK>(P, b, kvh, rt, ctx, qv[0], rowlen[0]);
    const int min_rowlen = P.causal ? ctx - (P.q_len - 1 - (rt * 16) / P.group) : ctx;
    f32x4_t acc[1][DVS][8];
#pragma unroll
    for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) acc[0][ds][jj] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    f32x4_t lacc[1] = {(f32x4_t){0.f, 0.f, 0.f, 0.f}};
    float m_run[1] = {kNegClamp}, f_run[1] = {kNegClamp};
    unpipelined_blocks<BS, DK, DV, ET, APPEND>(P, b, kvh, rt, ctx, blk_begin, blk_begin, blk_end, qv, rowlen,
                                               min_rowlen, acc, lacc, m_run, f_run);
    finish_segment<DV, OutT>(P, b, kvh, rt, nblk, blk_begin, blk_end, part_o, part_ml, acc[0], lacc[0], m_run[0],
                             f_run[0], 1.f);
}

// KV8: K and V caches hold E4M3FN bytes with one fp32 scale per (block, kv
// head). They are widened to bf16 in registers (exact) right before the
// MFMAs. The K scale folds into the softmax scale. The V scale is carried as
// the accumulator's frame: A is kept in units of the V scale of the last block
// it absorbed, and moving to a block with another scale multiplies the
// rescale factor by old/new. Each K load then reads 16 dims (16 bytes) of a
// token, so the QK contraction visits dims in a permuted order: k-step kk of
// lane group qd holds dims 16·qd + 64·(kk/2) + 8·(kk%2) .. +7, and Q is loaded
// in the same order.
//
// KLDS (16-bit caches, DK = 128): K is read like V, as whole 256-byte token
// rows (lane (qd, pc) reads 16-byte chunk pc of token 4qd+e of each 16-token
// tile, so one instruction covers four full rows; a compute unit's load path
// moves such rows about four times faster than the half-line reads of the
// register layout), with non-temporal loads (plain loads for sibling waves),
// and is rearranged into the QK operand layout through this wave's
// BS x 256-byte LDS buffer `klds`. Chunk c of token T sits at slot c ^ (T & 15) of the token's
// LDS row, so the row writes and the operand reads each touch 16 distinct
// 16-byte slots per 16 lanes. The K registers are free once a block is in
// LDS, so the next block's K is issued before this block's QK.
//
// ctx and nblk are sequence b's (clamped) context length and block count.
// ET: the element type of the query and bf16/fp16 caches (fp8 caches widen
// to bf16, so KV8 takes ET = bf16).
template <int BS, int DK, int DV, typename OutT, bool V_SHARED, bool KV8, bool KLDS = false, typename ET = __bf16,
          bool APPEND = false, int RTW = 1>
__device__ __forceinline__ void run_segment(const KernelParams &P, const int b, const int kvh, const int rt,
                                            const int ctx, const int nblk, const int blk_begin, const int blk_end,
                                            float *const part_o, float *const part_ml,
                                            const bool sync_siblings, char *const klds = nullptr) {
    constexpr int NT = BS / 16;            // 16-token tiles per KV block
    constexpr int KS = (DK + 31) / 32;     // 32-dim k-steps of QK
    constexpr int DVS = (DV + 127) / 128;  // 128-dim column sets of PV
    constexpr int ESZ = KV8 ? 1 : 2;       // cache element bytes
    static_assert(!KV8 || (DK % 64 == 0 && DV % 128 == 0), "fp8 caches: head dims multiple of 64 (K), 128 (V)");
    static_assert(!KLDS || (!KV8 && DK == 128), "K through LDS: 16-bit caches, DK = 128");
    static_assert(!KV8 || std::is_same<ET, __bf16>::value, "fp8 caches widen to bf16");
    static_assert(!(KV8 && APPEND), "fused append: 16-bit caches");
    static_assert(RTW == 1 || KLDS, "two row tiles per wave: K through LDS");
    const int lane = threadIdx.x & 63;
    const int qd = lane >> 4;
    const int pc = lane & 15;

    // ---- Q^T operand (row pc, dims 32kk+8qd..) and this row's visible
    // length, for each of the wave's RTW row tiles rt, rt+1, .. ----
    int rowlen[RTW];
    u32x4_t qv[RTW][KS];
#pragma unroll
    for (int r = 0; r < RTW; ++r) {
        rowlen[r] = 0;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) qv[r][kk] = (u32x4_t){0u, 0u, 0u, 0u};
        if (pc < min(16, P.rows - (rt + r) * 16)) {
            const int row = (rt + r) * 16 + pc;
            const int i = row / P.group, hh = row - i * P.group;
            const uint16_t *qrow = P.q + ((int64_t)(b * P.q_len + i) * P.num_heads + kvh * P.group + hh) * DK;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                const int dim = KV8 ? 16 * qd + 64 * (kk >> 1) + 8 * (kk & 1) : 32 * kk + 8 * qd;
                if (DK % 32 == 0 || dim < DK) qv[r][kk] = ld16(qrow + dim);
            }
            rowlen[r] = P.causal ? ctx - (P.q_len - 1 - i) : ctx;
        }
    }
    // shortest visible length over the valid rows of the wave's tiles
    // (wave-uniform; the first tile's first row): blocks that end at or before
    // it need no masking.
    const int min_rowlen = P.causal ? ctx - (P.q_len - 1 - (rt * 16) / P.group) : ctx;

    // Block-table entries are read through the scalar cache (constant address
    // space): the load is counted by lgkmcnt, so waiting for it never waits for
    // the K/V loads in flight. (A vector load issued after V(i) and needed for
    // K(i+1) would make the K(i+1) loads wait for all of V(i).)
    const __attribute__((address_space(4))) int32_t *bt_row =
        (const __attribute__((address_space(4))) int32_t *)(P.block_table + (int64_t)b * P.max_blocks);

    f32x4_t acc[RTW][DVS][8];
    // Row sums of the rounded p on the matrix unit (P x ones), kept in A's
    // frame: every lane holds rows 4qd+e like A's columns.
    f32x4_t lacc[RTW];
    float m_run[RTW], f_run[RTW];
#pragma unroll
    for (int r = 0; r < RTW; ++r) {
#pragma unroll
        for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) acc[r][ds][jj] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
        lacc[r] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
        m_run[r] = kNegClamp;
        f_run[r] = kNegClamp;
    }
    const u32x2_t ones4 = (u32x2_t){Elem<ET>::kOnePair, Elem<ET>::kOnePair};  // 1.0 of the element type
    constexpr float kLog2e = 1.4426950408889634f;

    // bf16: the operands themselves; fp8: the raw bytes (half the registers)
    u32x4_t kreg[NT][KV8 ? KS / 2 : KS];
    u32x4_t vreg[NT][DVS][KV8 ? 1 : 4];
    u32x2_t vraw[NT][DVS][KV8 ? 4 : 1];
    float vs_frame = 1.f;  // KV8: the V scale A is expressed in (this lane's row)

    // Addresses: a wave-uniform byte base plus one 32-bit per-lane offset that
    // is the same for every block.
    const int64_t k_tok_b = P.k_token_stride * ESZ, v_tok_b = P.v_token_stride * ESZ;
    const uint32_t k_lane = KLDS ? (uint32_t)(4 * qd * k_tok_b + 16 * pc) : (uint32_t)(pc * k_tok_b + 16 * qd);
    uint32_t kw_off[4], kr_off[KS];  // KLDS: LDS byte offsets of this lane's row writes / operand reads
    if constexpr (KLDS) {
#pragma unroll
        for (int e = 0; e < 4; ++e) kw_off[e] = (4 * qd + e) * 256 + ((pc ^ (4 * qd + e)) << 4);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) kr_off[kk] = pc * 256 + (((4 * kk + qd) ^ pc) << 4);
    }
    const uint32_t v_lane = (uint32_t)(4 * qd * v_tok_b + 8 * ESZ * pc);
    const char *k_head = reinterpret_cast<const char *>(P.k) + (int64_t)kvh * P.k_head_stride * ESZ;
    const char *v_head = reinterpret_cast<const char *>(P.v) + (int64_t)kvh * P.v_head_stride * ESZ;

    auto checked = [&](int phys, bool &bad) -> int {
        bad = (unsigned)phys >= (unsigned)P.num_pool_blocks;
        return bad ? 0 : phys;
    };
    // Base of 16-token tile t of block blk: tiles wholly past the context's end
    // read the zero page instead (the same lane offsets, L2-resident zeros), so
    // a sequence's last block costs only its valid tiles of HBM traffic while
    // the loads stay unconditional (their wait counts stay exact). Scores of
    // those tokens are masked and their V rows zeroed as before.
    auto tile_base = [&](const char *blk_base, int blk, int t, int64_t tok_b) -> const char * {
        const bool past = P.zero_page && 16 * t >= ctx - blk * BS;
        return past ? P.zero_page : blk_base + (int64_t)(16 * t) * tok_b;
    };
    auto load_k = [&](auto &kdst, int phys, int blk) {
        const char *kb = k_head + (int64_t)phys * P.k_block_stride * ESZ;
        if constexpr (KLDS) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const char *tb = tile_base(kb, blk, t, k_tok_b);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const char *kt = tb + (int64_t)e * k_tok_b + k_lane;
                    kdst[t][e] = V_SHARED ? *reinterpret_cast<const u32x4_t *>(kt) : stream_ld16(kt);
                }
            }
            return;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const char *kt = tile_base(kb, blk, t, k_tok_b);
#pragma unroll
            for (int kk = 0; kk < (KV8 ? KS / 2 : KS); ++kk) {
                if (KV8 || DK % 32 == 0 || 32 * kk + 8 * qd < DK)
                    kdst[t][kk] = *reinterpret_cast<const u32x4_t *>(kt + k_lane + 64 * kk);
                else
                    kdst[t][kk] = (u32x4_t){0u, 0u, 0u, 0u};
            }
        }
    };
    auto load_v_tile = [&](auto &vdst, auto &vrawdst, int phys, int blk, int t) {
        const char *vb = v_head + (int64_t)phys * P.v_block_stride * ESZ;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const char *vt = tile_base(vb, blk, t, v_tok_b) + (int64_t)e * v_tok_b;
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds) {
                    if constexpr (KV8) {
                        const u32x2_t *src = reinterpret_cast<const u32x2_t *>(vt + v_lane + 128 * ds);
                        vrawdst[t][ds][e] = V_SHARED ? *src : __builtin_nontemporal_load(src);
                    } else if (DV % 128 == 0 || 128 * ds + 8 * pc < DV) {
                        vdst[t][ds][e] = V_SHARED ? *reinterpret_cast<const u32x4_t *>(vt + v_lane + 256 * ds)
                                                  : stream_ld16(vt + v_lane + 256 * ds);
                    } else {
                        vdst[t][ds][e] = (u32x4_t){0u, 0u, 0u, 0u};
                    }
                }
            }
    };
    auto load_v = [&](auto &vdst, auto &vrawdst, int phys, int blk) {
#pragma unroll
        for (int t = 0; t < NT; ++t) load_v_tile(vdst, vrawdst, phys, blk, t);
    };

    // One KV block: QK on kr (or the LDS copy), softmax, PV on vr / vrw.
    // before_qk and after_qk place the single-buffer pipeline's loads of the
    // next block's K.
    auto compute_block = [&](const int blk, const int phys_b, const bool blk_bad, auto &kr, auto &vr, auto &vrw,
                             auto &&before_qk, auto &&after_qk, auto &&after_pv_tile) {
        const bool first = (blk == blk_begin);
        if (blk_bad && lane == 0) atomicOr(P.error_flag, kErrBadBlock);
        float sc = P.scale, vs = 1.f;
        if constexpr (KV8) {  // this block's dequantisation scales (wave-uniform, scalar loads)
            typedef const __attribute__((address_space(4))) float *cfloat_p;
            const int64_t si = (int64_t)phys_b * P.kv_heads + kvh;
            sc = P.scale * ((cfloat_p)P.k_scale)[si];
            vs = ((cfloat_p)P.v_scale)[si];
        }
        __builtin_amdgcn_sched_barrier(0);
        before_qk();

        const int blk0 = blk * BS;
        const bool full = !blk_bad && (blk0 + BS <= min_rowlen);
        const bool v_zero = KV8 && vs == 0.f;  // this block's V is zero: nothing to add
        // For scale > 0 the max of the scaled scores is the scaled max, so the
        // scale folds into the exponent below; otherwise scores are scaled first.
        const bool prescale = !(sc > 0.f);
        const float scl = prescale ? 1.f : sc;
        u32x2_t pa[RTW][NT];
        // row tile by row tile (one tile's scores live at a time; a second
        // tile reads K from LDS again)
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
            // ---- QK: S^T tiles ----
            f32x4_t s[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                f32x4_t c = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < KS; ++kk) {
                    u32x4_t kop;
                    if constexpr (KV8) {
                        const u32x4_t raw = kr[t][kk >> 1];
                        kop = (kk & 1) ? fp8x8_to_bf16x8(raw[2], raw[3]) : fp8x8_to_bf16x8(raw[0], raw[1]);
                    } else if constexpr (KLDS) {
                        kop = lds_ld16(klds, t * 4096 + kr_off[kk]);
                    } else {
                        kop = kr[t][kk];
                    }
                    c = Elem<ET>::mma32(kop, qv[r][kk], c);
                }
                s[t] = c;
            }
            if (r == 0) {
                __builtin_amdgcn_sched_barrier(0);
                after_qk();
                __builtin_amdgcn_sched_barrier(0);
            }

            // ---- softmax prepare: mask, block max of s*scale (golden :145-165) ----
            if (prescale) {
#pragma unroll
                for (int t = 0; t < NT; ++t) s[t] *= sc;
            }
            const int rvalid = blk_bad ? 0 : rowlen[r] - blk0;  // tokens of this block visible to row pc
            // one wave-uniform branch around the masking (per-element selects
            // would run on every block)
            if (!full) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (16 * t + 4 * qd + e >= rvalid) s[t][e] = -INFINITY;
            }
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[t][e]);
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mb = fmaxf(mx * scl, kNegClamp);

            // ---- online merge coefficients (aiv_online_update.cpp:183-207) ----
            const float mnew = first ? mb : fmaxf(m_run[r], mb);
            const bool use = first || (mb >= mnew - kFrameGap);
            const float cfe = first ? 0.f : (use ? __expf(f_run[r] - mb) : 1.f);  // e^{f - m_blk}
            float cf = cfe;
            if (KV8 && use && !v_zero) {  // move this row's A into the block's V-scale frame
                cf *= vs_frame / vs;
                vs_frame = vs;
            }

            // ---- p = bf16(exp(s*scale - m_blk)) = bf16(exp2(s*scale*log2e -
            // m_blk*log2e)); a skipped block (use false) gives p = 0 ----
            const float mb2 = use ? mb * kLog2e : INFINITY;
            const float sc2 = scl * kLog2e;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float p[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][e], sc2, -mb2));
                pa[r][t] = (u32x2_t){Elem<ET>::pack2(p[0], p[1]), Elem<ET>::pack2(p[2], p[3])};
            }
            m_run[r] = mnew;
            if (use) f_run[r] = mb;

            // ---- rescale A (and its row sums) to the new frame (rows 4qd+e
            // live in lane 4qd+e's factors) ----
            {
                f32x4_t cv, cl;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    cv[e] = __shfl(cf, 4 * qd + e, 64);
                    cl[e] = KV8 ? __shfl(cfe, 4 * qd + e, 64) : cv[e];
                }
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) acc[r][ds][jj] *= cv;
                lacc[r] *= cl;
            }
            // row sums of the rounded p (every column of P x ones is the
            // sum), also for a block whose V adds nothing
            if constexpr (kTilePairs<NT, RTW>) {
#pragma unroll
                for (int t = 0; t < NT; t += 2)
                    lacc[r] = mma_tile_pair<ET>(pa[r][t], pa[r][t + 1], ones4, ones4, lacc[r]);
            } else {
#pragma unroll
                for (int t = 0; t < NT; ++t) lacc[r] = Elem<ET>::mma16(pa[r][t], ones4, lacc[r]);
            }
        }

        // ---- PV: A += P * V ----
        const int vvalid = (blk_bad || v_zero) ? 0 : min(BS, ctx - blk0);  // tokens with defined V
        // V rows past the context's end (and of an out-of-pool block) are
        // zeroed once, under one wave-uniform branch ahead of PV, where the
        // selects would run on every block. The K-through-LDS kernel keeps
        // them in PV, which measured faster there (cfg2: 112.5 against
        // 113.2 us per step; fp8 63.1 against 62.8 the other way).
        constexpr bool kZeroAhead = !KLDS;
        if (kZeroAhead && vvalid < BS) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (16 * t + 4 * qd + e >= vvalid)
#pragma unroll
                        for (int ds = 0; ds < DVS; ++ds) {
                            if constexpr (KV8)
                                vrw[t][ds][e] = (u32x2_t){0u, 0u};
                            else
                                vr[t][ds][e] = (u32x4_t){0u, 0u, 0u, 0u};
                        }
        }
        if constexpr (kTilePairs<NT, RTW>) {  // two token tiles per PV MFMA
            // V^T operand words of token tile t: the bf16 of dim 2w + (jj & 1) of
            // tokens (0, 1) and (2, 3) of lane (pc, qd)'s four rows 4qd + e, low
            // halves (bytes 0-1 of each) or high halves (bytes 2-3), one v_perm_b32
            // each (bytes 0-3 from the second operand, 4-7 from the first)
            auto v_words = [&](const u32x4_t (&vt4)[4], const int jj) -> u32x2_t {
                const int w = jj >> 1;
                constexpr unsigned kLoHalves = 0x05040100u, kHiHalves = 0x07060302u;
                const unsigned sel = (jj & 1) ? kHiHalves : kLoHalves;
                return (u32x2_t){__builtin_amdgcn_perm(vt4[1][w], vt4[0][w], sel),
                                 __builtin_amdgcn_perm(vt4[3][w], vt4[2][w], sel)};
            };
            // tile t's V rows (8 bf16 dims of tokens 16t + 4qd + e), rows past
            // vvalid zeroed
            auto v_tile = [&](const int t, u32x4_t (&vt4)[DVS][4]) {
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (KV8)
                            vt4[ds][e] = fp8x8_to_bf16x8(vrw[t][ds][e][0], vrw[t][ds][e][1]);
                        else
                            vt4[ds][e] = vr[t][ds][e];
                    }
                if (!kZeroAhead && vvalid < BS) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (16 * t + 4 * qd + e >= vvalid)
#pragma unroll
                            for (int ds = 0; ds < DVS; ++ds) vt4[ds][e] = (u32x4_t){0u, 0u, 0u, 0u};
                }
            };
            constexpr int TP = 2;  // token tiles per PV MFMA (mma_tile_pair)
#pragma unroll
            for (int t = 0; t < NT; t += TP) {
              if (!(KV8 && v_zero)) {  // wave-uniform: a zero-scale block adds nothing
                u32x4_t vt4[TP][DVS][4];
#pragma unroll
                for (int u = 0; u < TP; ++u) v_tile(t + u, vt4[u]);
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const u32x2_t b0 = v_words(vt4[0][ds], jj), b1 = v_words(vt4[1][ds], jj);
#pragma unroll
                        for (int r = 0; r < RTW; ++r)
                            acc[r][ds][jj] = mma_tile_pair<ET>(pa[r][t], pa[r][t + 1], b0, b1, acc[r][ds][jj]);
                    }
              }
#pragma unroll
                for (int u = 0; u < TP; ++u) after_pv_tile(t + u);
            }
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              if (!(KV8 && v_zero)) {  // wave-uniform: a zero-scale block adds nothing
                u32x4_t vt4[DVS][4];       // 8 bf16 dims of tokens 16t + 4qd + e
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (KV8)
                            vt4[ds][e] = fp8x8_to_bf16x8(vrw[t][ds][e][0], vrw[t][ds][e][1]);
                        else
                            vt4[ds][e] = vr[t][ds][e];
                    }
                if (!kZeroAhead && vvalid < BS) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (16 * t + 4 * qd + e >= vvalid)
#pragma unroll
                            for (int ds = 0; ds < DVS; ++ds) vt4[ds][e] = (u32x4_t){0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const int w = jj >> 1;
                        const unsigned a0 = vt4[ds][0][w], a1 = vt4[ds][1][w];
                        const unsigned a2 = vt4[ds][2][w], a3 = vt4[ds][3][w];
                        // the bf16 of dim 2w + (jj & 1) of tokens (0, 1) and (2, 3):
                        // low halves (bytes 0-1 of each) or high halves (bytes 2-3),
                        // one v_perm_b32 each (bytes 0-3 from the second operand,
                        // 4-7 from the first)
                        constexpr unsigned kLoHalves = 0x05040100u, kHiHalves = 0x07060302u;
                        const unsigned sel = (jj & 1) ? kHiHalves : kLoHalves;
                        const unsigned d0 = __builtin_amdgcn_perm(a1, a0, sel);
                        const unsigned d1 = __builtin_amdgcn_perm(a3, a2, sel);
#pragma unroll
                        for (int r = 0; r < RTW; ++r)
                            acc[r][ds][jj] = Elem<ET>::mma16(pa[r][t], (u32x2_t){d0, d1}, acc[r][ds][jj]);
                    }
              }
                after_pv_tile(t);
            }
        }
    };

    // Per block i: V(i) is issued first, then QK(i) consumes K(i) (issued
    // during block i-1), then K(i+1) is issued (with K staged through LDS: as
    // soon as K(i) is in LDS, before QK(i)), then softmax and PV(i). fp8
    // caches (kRefillV) issue V(i+1) earlier instead: as PV(i) finishes with
    // V(i)'s token tile t, V(i+1)'s tile t goes into the same registers, so V
    // stays in flight through the math without a second register set (fp8
    // cfg2 shape 58.8 against 59.5-59.7 us; neutral for 16-bit caches and
    // 1.3% slower for sibling waves). The scheduling barriers keep the
    // compiler from sinking loads past the math, which would serialise the
    // memory latency. The segment's last block is peeled off (no K(i+1),
    // V(i+1)): with the prefetch under a run-time condition the compiler's
    // wait counts would have to cover the path without it, so PV(i) would wait
    // for K(i+1) as well.
    constexpr bool kRefillV = KV8;
    bool bad = false;
    int phys = checked(bt_row[blk_begin], bad);
    auto step = [&](const int blk, auto has_next) {
        constexpr bool NEXT = decltype(has_next)::value;
        const bool blk_bad = bad;
        const int phys_b = phys;
        const int raw_next = NEXT ? bt_row[blk + 1] : 0;  // in flight during this block's loads
        __builtin_amdgcn_sched_barrier(0);
        // Sibling waves (row tiles of one kv head) read the same K/V: issuing a
        // block's loads together lets the caches serve the second request.
        if (V_SHARED && sync_siblings) __builtin_amdgcn_s_barrier();
        if constexpr (!kRefillV) load_v(vreg, vraw, phys_b, blk);
        auto stage_k_and_prefetch = [&] {
            if constexpr (KLDS) {
                // K(i) into LDS (waits for it; V(i) stays in flight), then K(i+1) into the freed registers
                wave_lds_sync();
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) lds_st16(klds, t * 4096 + kw_off[e], kreg[t][e]);
                wave_lds_sync();
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (NEXT) {
                    phys = checked(raw_next, bad);
                    load_k(kreg, phys, blk + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        auto prefetch_k = [&] {
            if constexpr (!KLDS && NEXT) {
                phys = checked(raw_next, bad);
                load_k(kreg, phys, blk + 1);
            }
        };
        auto refill_v = [&](int t) {  // after PV(i) of token tile t; phys is block i+1's by then
            if constexpr (kRefillV && NEXT) load_v_tile(vreg, vraw, phys, blk + 1, t);
        };
        compute_block(blk, phys_b, blk_bad, kreg, vreg, vraw, stage_k_and_prefetch, prefetch_k, refill_v);
    };
    // blocks [blk_begin, end), end > blk_begin, through the pipeline
    auto pipeline = [&](const int end) {
        load_k(kreg, phys, blk_begin);
        if constexpr (kRefillV) load_v(vreg, vraw, phys, blk_begin);
        for (int blk = blk_begin; blk + 1 < end; ++blk) step(blk, std::true_type{});
        step(end - 1, std::false_type{});
    };
    if constexpr (APPEND) {
        // Fused append: the blocks from the first one holding a new token on
        // run after the pipeline, in unpipelined_blocks, which reads the new
        // rows there. (Kept apart from the plain decode's path: a run-time
        // condition around the pipeline's first load would loosen the
        // compiler's wait counts in the loop.)
        const int pipe_end = max(blk_begin, min(blk_end, ctx - P.q_len < 0 ? 0 : (ctx - P.q_len) / BS));
        if (pipe_end > blk_begin) pipeline(pipe_end);
        if (pipe_end < blk_end)
            unpipelined_blocks<BS, DK, DV, ET, true, RTW>(P, b, kvh, rt, ctx, blk_begin, pipe_end, blk_end, qv, rowlen,
                                                          min_rowlen, acc, lacc, m_run, f_run);
    } else {
        pipeline(blk_end);
    }

    // tile rt + r's pieces sit r pieces-of-a-worker-wave further on (two slots each)
#pragma unroll
    for (int r = 0; r < RTW; ++r)
        finish_segment<DV, OutT>(P, b, kvh, rt + r, nblk, blk_begin, blk_end, part_o + r * (2 * 16 * DV),
                                 part_ml + r * (2 * 32), acc[r], lacc[r], m_run[r], f_run[r], vs_frame);
}

// ---------------------------------------------------------------------------
// Main kernel: one wavefront per wave slot, one equal slice of the work each
// ---------------------------------------------------------------------------

// MAXW = 1: one wave per worker (one row tile per kv head); MAXW = 4: up to
// four sibling waves, one per row tile, walk the same KV blocks, so V is loaded
// through the caches (the siblings hit each other's lines) rather than
// streamed past them.
// RTW = 2 (with MAXW = 1): one wave runs both row tiles of a row group,
// every K and V operand feeding the two tiles' MFMAs.
template <int BS, int DK, int DV, typename OutT, int MAXW, bool KV8 = false, typename ET = __bf16,
          bool APPEND = false, int RTW = 1>
__global__ void __launch_bounds__(64 * MAXW) pa_decode_kernel(const KernelParams P) {
    static_assert(BS % 16 == 0 && BS >= 16 && BS <= 128, "block_size must be 16..128, multiple of 16");
    static_assert(DK % 8 == 0 && DV % 8 == 0, "head dims must be multiples of 8");
    static_assert(!KV8 || BS * DK <= 16384, "fp8 caches: blocks that fit the registers");
    // 16-bit caches with 128-dim heads stage K through LDS, BS x 256 bytes per
    // wave: a static buffer for single-wave workers, the launch's dynamic LDS
    // (one buffer per sibling wave of the workgroup) otherwise
    constexpr bool KLDS = !KV8 && DK == 128;
    __shared__ __attribute__((aligned(16))) char klds1[(KLDS && MAXW == 1) ? BS * 256 : 16];
    extern __shared__ __attribute__((aligned(16))) char klds_waves[];
    flag_bad_lengths(P);
    const int w = blockIdx.x;
    const int wave = MAXW == 1 ? 0 : (int)(threadIdx.x >> 6);
    char *const klds = MAXW == 1 ? klds1 : klds_waves + wave * (BS * 256);
    const int tpb = lane_tiles(P);
    const int list = w % P.lanes;
    int start = 0, end = 0, b = 0, prefix = 0, ctx0 = 0;
    locate_slice(P, w / P.lanes, &start, &end, &b, &prefix, &ctx0);
    // wave-uniform values (cross-lane results), kept in scalar registers so that
    // block-table and scale reads derived from them are scalar loads
    start = __builtin_amdgcn_readfirstlane(start);
    end = __builtin_amdgcn_readfirstlane(end);
    b = __builtin_amdgcn_readfirstlane(b);
    prefix = __builtin_amdgcn_readfirstlane(prefix);
    if (start >= end) return;
    int ctx = __builtin_amdgcn_readfirstlane(ctx0);  // the segment's sequence
    int nb = (ctx + BS - 1) / BS;
    if (nb == 0) return;  // not reached: the batch holding `start` has work
    const int rel = start - prefix;
    int j = rel / nb;
    int blk = rel - j * nb;
    int pos = start;
    int slot = 0;
    while (pos < end && nb > 0) {
        const int seg = min(end - pos, nb - blk);
        const int jt = list_tile0(P, list, b) + j;  // tile of the batch
        const int kvh = jt / P.row_groups, rg = jt - kvh * P.row_groups;
        const int rt = rg * P.tiles_per_worker + wave;  // this wave's row tile
        // A worker touches at most two tiles partially: the first and the last
        // of its slice (slots 0 and 1); tiles in between are finished here.
        const int64_t piece = ((int64_t)w * P.tiles_per_worker + wave) * 2 + slot;
        float *po = P.part_o + piece * 16 * DV;
        float *pml = P.part_ml + piece * 32;
        // every wave of the group has a row tile: all run the same blocks, so
        // a per-block barrier among them is matched
        const bool full_group = (rg + 1) * P.tiles_per_worker <= P.row_tiles;
        if (rt < P.row_tiles) {
            if constexpr (BS * DK > 16384 || BS * DV > 16384)  // a block's K or V exceeds the registers
                run_segment_big<BS, DK, DV, OutT, ET, APPEND>(P, b, kvh, rt, ctx, nb, blk, blk + seg, po, pml);
            else
                run_segment<BS, DK, DV, OutT, (MAXW > 1), KV8, KLDS, ET, APPEND, RTW>(
                    P, b, kvh, rt, ctx, nb, blk, blk + seg, po, pml, MAXW > 1 && full_group, klds);
        }
        pos += seg;
        slot = 1;
        if (pos >= end) break;
        blk = 0;
        if (++j == tpb) {
            j = 0;
            do {
                ++b;
                ctx = __builtin_amdgcn_readfirstlane(ctx_of(P, b));
                nb = (ctx + BS - 1) / BS;
            } while (nb == 0 && b + 1 < P.batch);
        }
    }
}

// ---------------------------------------------------------------------------
// Merge kernel: one workgroup per tile; log-sum-exp merge of the pieces
// (pa_kernel.cce:1666-1773 CombineScale), and zeros for empty contexts.
// ---------------------------------------------------------------------------

// Threads per merge workgroup: one 16-byte unit of a tile's 16 x DV output per
// thread up to DV = 128 (512 threads), four per thread for MLA's DV = 512.
template <int DV> constexpr int merge_threads() { return DV * 4 < 512 ? (DV * 4 < 64 ? 64 : DV * 4) : 512; }
constexpr int kMergeLdsPieces = 32;  // pieces per tile merged through LDS weights

template <int DV, typename OutT>
// MLA (DV = 512): every tile of a launch is cut, and 1024 of them (cfg4) fit
// the chip at once only at eight waves per SIMD, i.e. 64 registers, hence one
// piece read ahead (measured 24.9 -> 23.2 us against four waves per SIMD with
// four read ahead).
__global__ void __launch_bounds__(merge_threads<DV>()) __attribute__((amdgpu_waves_per_eu(DV >= 512 ? 8 : 1)))
pa_merge_kernel(const KernelParams P) {
    constexpr int MT = merge_threads<DV>();
    constexpr int UNITS = 16 * (DV / 4);        // 16-byte units of a full tile
    constexpr int UPT = (UNITS + MT - 1) / MT;  // units per thread
    constexpr int PRE = UPT == 1 ? 8 : (DV >= 512 ? 1 : 4);  // pieces per unit read before the weights are known
    const int tid = threadIdx.x;
    // The main kernel is done: hand its error word to the host through
    // pinned memory (a run's wait then needs no device-to-host copy).
    if (P.err_mirror && blockIdx.x == 0 && tid == 0)
        __hip_atomic_store(P.err_mirror, __hip_atomic_load(P.error_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int tpb = P.kv_heads * P.row_tiles;
    const int tile = blockIdx.x;  // (batch, kv head, row tile)
    const int b = tile / tpb, jr = tile - b * tpb;
    const int kvh = jr / P.row_tiles, rt = jr - kvh * P.row_tiles;
    const int rg = rt / P.tiles_per_worker, wave = rt - rg * P.tiles_per_worker;
    const int jt = kvh * P.row_groups + rg;  // tile of the batch in the work lists
    const int list = list_of_tile(P, jt / lane_tiles(P), b), j = jt - (jt / lane_tiles(P)) * lane_tiles(P);
    const int rows_here = min(16, P.rows - rt * 16);
    int prefix = 0;
    int ctxb = 0;
    const int total = scan_work(P, b, &prefix, &ctxb, -1, nullptr, nullptr, nullptr);
    const int nb = (ctxb + P.block_size - 1) / P.block_size;
    if (nb == 0) {  // empty context: defined as a zero output
        for (int idx = tid; idx < rows_here * (DV / 4); idx += MT) {
            const int row = idx / (DV / 4), c4 = idx - row * (DV / 4);
            OutStore<OutT>::store4(P.out, out_row_offset(P, b, kvh, rt * 16 + row, DV) + 4 * c4,
                                   (f32x4_t){0.f, 0.f, 0.f, 0.f});
        }
        return;
    }
    const int per_list = max(P.workers / P.lanes, 1);
    const int chunk = (total + per_list - 1) / per_list;
    const int t0 = prefix + j * (nb + P.seg_cost);  // the tile's first work unit
    const int tb = t0 + P.seg_cost;                 // its first block's
    const int w_first = tb / chunk, w_last = (tb + nb - 1) / chunk;  // slices of the list
    if (w_first == w_last) return;  // a tile inside one slice is finished by the main kernel
    // Log-sum-exp over the pieces: the row max and total l from the (m, l)
    // pairs first, then O = sum_w e^{m_w - M} O_w / L, whose piece loads do not
    // depend on each other and stay in flight together.
    auto piece_of = [&](int c) -> int64_t {
        const int slot = (c * chunk >= t0) ? 0 : 1;
        const int64_t w = (int64_t)c * P.lanes + list;  // the worker that ran slice c
        return (w * P.tiles_per_worker + wave) * 2 + slot;
    };
    const int np = w_last - w_first + 1;
    if (np <= kMergeLdsPieces) {
        // Per-(row, piece) weights e^{m_w - M} / L once per workgroup, then the
        // partial rows stream through with no dependent loads in the way. Every
        // unit of the thread has its first PRE pieces read together with the
        // (m, l) loads: they do not depend on the weights, so the merge is one
        // memory round trip after the work scan, not one per unit.
        __shared__ float wgt[16][kMergeLdsPieces];  // m of each (row, piece), then its weight
        __shared__ float lsum[16][kMergeLdsPieces];
        const int units = rows_here * (DV / 4);
        f32x4_t pre[UPT][PRE];
#pragma unroll
        for (int u = 0; u < UPT; ++u) {
            const int idx = tid + u * MT;
            const int row = idx / (DV / 4), c4 = idx - row * (DV / 4);
#pragma unroll
            for (int k = 0; k < PRE; ++k)
                pre[u][k] = (idx < units && k < np)
                                ? *reinterpret_cast<const f32x4_t *>(P.part_o + (piece_of(w_first + k) * 16 + row) * DV +
                                                                     4 * c4)
                                : (f32x4_t){0.f, 0.f, 0.f, 0.f};
        }
        for (int e = tid; e < 16 * np; e += MT) {  // all (m, l) loads in flight at once
            const int row = e / np, k = e - row * np;
            const int64_t pc = piece_of(w_first + k);
            wgt[row][k] = P.part_ml[pc * 32 + row];
            lsum[row][k] = P.part_ml[pc * 32 + 16 + row];
        }
        __syncthreads();
        if (tid < 16) {
            float M = -INFINITY;
            for (int k = 0; k < np; ++k) M = fmaxf(M, wgt[tid][k]);
            float L = 0.f;
            for (int k = 0; k < np; ++k) {
                const float c = __expf(wgt[tid][k] - M);
                wgt[tid][k] = c;
                L += c * lsum[tid][k];
            }
            const float inv = L > 0.f ? 1.f / L : 0.f;
            for (int k = 0; k < np; ++k) wgt[tid][k] *= inv;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < UPT; ++u) {
            const int idx = tid + u * MT;
            if (idx >= units) break;
            const int row = idx / (DV / 4), c4 = idx - row * (DV / 4);
            f32x4_t o = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < PRE; ++k)
                if (k < np) o += wgt[row][k] * pre[u][k];
#pragma unroll 4
            for (int k = PRE; k < np; ++k) {
                const int64_t piece = piece_of(w_first + k);
                o += wgt[row][k] * *reinterpret_cast<const f32x4_t *>(P.part_o + (piece * 16 + row) * DV + 4 * c4);
            }
            OutStore<OutT>::store4(P.out, out_row_offset(P, b, kvh, rt * 16 + row, DV) + 4 * c4, o);
        }
        return;
    }
    for (int idx = tid; idx < rows_here * (DV / 4); idx += MT) {
        const int row = idx / (DV / 4), c4 = idx - row * (DV / 4);
        float M = -INFINITY;
        for (int w = w_first; w <= w_last; ++w) M = fmaxf(M, P.part_ml[piece_of(w) * 32 + row]);
        float L = 0.f;
        f32x4_t o = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
        for (int w = w_first; w <= w_last; ++w) {
            const int64_t piece = piece_of(w);
            const float c = __expf(P.part_ml[piece * 32 + row] - M);
            L += c * P.part_ml[piece * 32 + 16 + row];
            o += c * *reinterpret_cast<const f32x4_t *>(P.part_o + (piece * 16 + row) * DV + 4 * c4);
        }
        const f32x4_t res = L > 0.f ? o / L : (f32x4_t){0.f, 0.f, 0.f, 0.f};
        OutStore<OutT>::store4(P.out, out_row_offset(P, b, kvh, rt * 16 + row, DV) + 4 * c4, res);
    }
}


// ---------------------------------------------------------------------------
// MLA decode: one latent KV head shared by every query head (Hkv = 1 in the
// DeepSeek shape, Dk = 576, Dv = 512), V = the first Dv dims of K.
//
// A worker workgroup of four waves owns up to 128 query rows (a "row group",
// 32 rows per wave), so with 128 query heads each KV block of a work slice
// is fetched from HBM into LDS once, by one compute unit. Blocks are copied
// with direct global->LDS loads (double buffered: the next block is in flight
// during the math on this one). Each wave runs its 32 rows end to end; Q
// (Dk/16 operand quads) and O^T (Dv x 32 rows, fp32) stay in its registers,
// and the waves share only the block buffers.
//   QK  S^T[token][row] = K[token][:] . Q[row][:]   MFMA 32x32x16 bf16,
//       A = K rows from LDS (16-B reads), B = Q registers. C: lane l holds
//       row l%32 and, in register 4a+e, token 8a+4h+e of the 32-token tile
//       (h = l/32).
//   PV  O^T[dim][row] += V^T[dim][token] . P^T[token][row]   MFMA 32x32x16,
//       A = V^T from LDS by transposing reads (ds_read_b64_tr_b16, two per
//       operand), B = P^T, which is the QK result layout itself: for the
//       16-token k-step s of a 32-token tile, registers 8s..8s+7 of lane l
//       hold tokens {16s+4h..16s+4h+3, 16s+8+4h..16s+8+4h+3}; the V^T reads
//       pick the same token order.
// Every lane of S^T and O^T holds a single query row, so the block max, the
// rescale and the row sum are per lane plus one exchange between the two lane
// halves. Numerics are the same per-block recipe as the decode kernel.
//
// LDS row layout: a token's Dk*2 bytes as 16-byte chunks, the row padded to a
// chunk count = 10 (mod 16): 74 chunks (1184 B) for Dk = 576. Measured on
// MI355X with the kernel's access patterns (per 16 lanes: 16 token rows x 16 B
// for K, 4 token rows x 32 B for the transposing V^T reads), that stride runs
// both at full LDS speed (534-548 and 420-427 B/ns per CU), where 73, 76 and
// 77 chunks, with or without XOR swizzles of the chunk index, halve one of
// them.
// ---------------------------------------------------------------------------

template <int DK>
struct MlaLayout {
    static constexpr int kChunks = DK / 8;                                           // 16-B chunks per token
    static constexpr int kRowChunks = kChunks + ((10 - kChunks % 16) % 16 + 16) % 16;  // = 10 (mod 16)
    static constexpr int kRowBytes = kRowChunks * 16;
};

__device__ __forceinline__ i16x4_t lds_ld_tr(const char *base, uint32_t off) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4_t *)((LDS_AS char *)base + off));
}

constexpr int kMlaRowsPerWave = 32;    // MFMA N of the 32x32x16 tiles
constexpr int kMlaRowsPerGroup = 128;  // four waves x 32 rows

__device__ __forceinline__ f32x16_t mma_32x32x16(const u32x4_t a, const u32x4_t b, const f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// Work slice and row group of workgroup w. Row groups of a slice are
// w, w+8, w+16, ...: the same XCD under round-robin workgroup dispatch.
__device__ __forceinline__ void mla_worker(int w, int slices, int groups, int *slice, int *group) {
    const int full = slices / 8;  // complete sets of 8 slices
    const int per_set = 8 * groups;
    const int set = w / per_set;
    if (set < full) {
        *slice = set * 8 + (w & 7);
        *group = (w / 8) % groups;
    } else {
        const int rem = slices - full * 8;  // > 0 here
        const int x = w - full * per_set;
        *slice = full * 8 + x % rem;
        *group = x / rem;
    }
}

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Buffer loads straight into LDS (lane l -> LDS base + size*l). Lanes whose
// offset is at or past the descriptor's record count are not fetched and
// write zeros. Issued as inline asm on purpose: the compiler's wait
// insertion would otherwise treat every later LDS read (the transposing reads
// in particular) as possibly aliasing the fill and wait for all outstanding
// vector memory before it, which serialises the next block's fill with this
// block's math. Completion is instead awaited explicitly (s_waitcnt vmcnt at
// the block barrier); loads the compiler does not count can only make its
// own vmcnt waits stricter, since vector memory completes in order.
// m0 holds the wave's LDS destination; nothing else in these kernels uses it.
// One wait state separates the m0 write from the LDS-DMA load that reads it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_fill16(i32x4_t rsrc, uint32_t voffset, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voffset), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ uint32_t lds_addr_of(const char *p) {
    return (uint32_t)(uintptr_t)(const LDS_AS char *)p;
}

// Raw buffer descriptor (stride 0, num_records in bytes). The values are
// wave-uniform; readfirstlane puts them in scalar registers so the load needs
// no per-lane descriptor loop.
__device__ __forceinline__ i32x4_t buffer_rsrc(const void *base, uint32_t num_records) {
    const uint64_t a = (uint64_t)base;
    return (i32x4_t){__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                     __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu)),
                     __builtin_amdgcn_readfirstlane((int)num_records), 0x00020000};
}

template <int BS, int DK, int DV, typename OutT>
__device__ __forceinline__ void run_mla_segment(const KernelParams &P, const int slice, const int rgrp, const int b,
                                                const int kvh, const int nblk, const int blk_begin, const int blk_end,
                                                const int slot, char *const smem0, char *const smem1) {
    using L = MlaLayout<DK>;
    constexpr int RB = L::kRowBytes;
    constexpr int RC = L::kRowChunks;
    constexpr int KC = L::kChunks;
    constexpr int NI = BS * RC / 64;   // 1 KB direct-to-LDS loads per block
    constexpr int NII = (NI + 3) / 4;  // of which each wave issues at most NII
    constexpr int KS = DK / 16;        // QK k-steps
    constexpr int NT = BS / 32;        // 32-token tiles
    constexpr int PS = BS / 16;        // PV k-steps
    constexpr int NM = DV / 32;        // O^T tiles of 32 dims
    static_assert(BS % 32 == 0 && (BS * RC) % 64 == 0, "block of whole 32-token tiles");
    static_assert(DK % 16 == 0 && DV % 32 == 0 && DV <= DK, "V is a prefix of K");

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int h = lane >> 5, j = lane & 31;  // lane half, query row of the wave
    const int r0 = rgrp * kMlaRowsPerGroup + kMlaRowsPerWave * wave;  // first query row of this wave
    const int rows_here = min(kMlaRowsPerWave, P.rows - r0);
    const bool active = rows_here > 0;  // wave-uniform
    const int ctx = min(max(P.context_lens[b], 0), P.max_blocks * BS);

    // ---- Q (B operand of QK): row j, dims 16kk+8h..+7 ----
    u32x4_t qv[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qv[kk] = (u32x4_t){0u, 0u, 0u, 0u};
    int rowlen = 0;
    if (j < rows_here) {
        const int r = r0 + j;
        const int i = r / P.group, hh = r - i * P.group;
        const uint16_t *qrow = P.q + ((int64_t)(b * P.q_len + i) * P.num_heads + kvh * P.group + hh) * DK + 8 * h;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) qv[kk] = ld16(qrow + 16 * kk);
        rowlen = P.causal ? ctx - (P.q_len - 1 - i) : ctx;
    }
    const int min_rowlen = P.causal ? ctx - (P.q_len - 1 - r0 / P.group) : ctx;

    // Block-table entries are read through the scalar cache (constant
    // address space): the load is counted by lgkmcnt, so waiting for it never
    // waits for the vector-memory loads in flight (the block fill).
    const __attribute__((address_space(4))) int32_t *bt_row =
        (const __attribute__((address_space(4))) int32_t *)(P.block_table + (int64_t)b * P.max_blocks);
    auto phys_of = [&](int blk, bool &bad) -> int {
        const int phys = bt_row[blk];
        bad = (unsigned)phys >= (unsigned)P.num_pool_blocks;
        return bad ? 0 : phys;
    };

    // ---- direct-to-LDS fill: LDS chunk p = 64*i + lane holds token p / RC,
    // chunk p % RC. The per-lane byte offsets within a KV block
    // are the same for every block; pad chunks re-read chunk 0 of their token.
    // The descriptor's record count (valid tokens x token bytes, 0 for an
    // out-of-pool block) makes every later token read zeros. ----
    const uint32_t tok_b = (uint32_t)(P.k_token_stride * 2);  // block bytes < 2^31 (host-checked)
    const char *k_head = reinterpret_cast<const char *>(P.k) + (int64_t)kvh * P.k_head_stride * 2;
    // Lane l of load ii fills LDS chunk p = 256 ii + 64 wave + l of the
    // buffer: token p / RC, chunk p % RC. Since 256 = 3 RC + 34 for RC = 74,
    // its byte offset in the block follows from the lane's first chunk
    // (token t0, chunk c0) as t0*tok + 16 c0 + ii (3 tok + 16*34) + k (tok -
    // 16 RC), k = (c0 + 34 ii) / RC, computed per load rather than held in
    // NII registers. Pad chunks (p % RC >= KC) fetch the first bytes of the
    // next token, or zeros past the descriptor's record count.
    constexpr int kStepChunks = 256 % RC;  // chunks past the whole rows a load index advances
    constexpr int kStepRows = 256 / RC;
    const int p0 = 64 * wave + lane;
    const int t0 = p0 / RC, c0 = p0 - (p0 / RC) * RC;
    const uint32_t fill_base = (uint32_t)t0 * tok_b + 16u * (uint32_t)c0;
    const uint32_t fill_step = (uint32_t)kStepRows * tok_b + 16u * kStepChunks;
    const uint32_t fill_wrap = tok_b - 16u * RC;  // one more whole row, less the chunks
    constexpr uint32_t kDivRC = (65536u + RC - 1) / RC;
    static_assert([] {
        for (uint32_t x = 0; x < RC + kStepChunks * NII; ++x)
            if ((x * kDivRC) >> 16 != x / RC) return false;
        return true;
    }(), "multiply-shift division by RC");
    // A block's fill as a buffer descriptor and an LDS
    // address, both wave-uniform; its loads are issued one at a time so that
    // those of the next block can be spread over this block's math (issued
    // in a burst, the four waves' loads queue behind each other at the
    // compute unit's vector-memory unit and stall every wave's issue).
    struct Fill {
        i32x4_t rsrc;
        uint32_t lds;
    };
    // blk < 0: a descriptor with no records, whose loads fetch nothing (and
    // write zeros to LDS): the loads stay unconditional, without branches in
    // the math and with a fixed count for the vmcnt waits.
    auto fill_of = [&](int blk, char *dst, bool &bad) -> Fill {
        bad = false;
        const int phys = blk >= 0 ? phys_of(blk, bad) : 0;
        const int vvalid = (bad || blk < 0) ? 0 : min(BS, ctx - blk * BS);
        return {buffer_rsrc(k_head + (int64_t)phys * P.k_block_stride * 2, (uint32_t)vvalid * tok_b),
                (uint32_t)__builtin_amdgcn_readfirstlane(lds_addr_of(dst) + 1024u * wave)};
    };
    // Per-lane offsets: recomputed for every block from two registers. The
    // empty asm hides that they do not change, so the compiler cannot hoist
    // NII offsets out of the block loop into registers it does not have.
    auto fill_regs = [&](uint32_t &base, uint32_t &cc) {
        base = fill_base;
        cc = (uint32_t)c0;
        asm volatile("" : "+v"(base), "+v"(cc));
    };
    auto fill_one = [&](const Fill &f, int ii, uint32_t base, uint32_t cc) {
        if (NI % 4 == 0 || 4 * ii + wave < NI) {
            // (cc + kStepChunks ii) / RC by a 24-bit multiply and shift, exact
            // over the operand's range (checked at compile time); k * wrap as
            // a signed 24-bit multiply-add (the host keeps |wrap| < 2^23)
            const uint32_t k = __umul24(cc + kStepChunks * ii, kDivRC) >> 16;
            const uint32_t off = (uint32_t)(__mul24((int)k, (int)fill_wrap) + (int)(base + ii * fill_step));
            lds_fill16(f.rsrc, off, f.lds + 4096u * ii);
        }
    };

    // O^T accumulators (tile mt: dims 32mt .. 32mt+31 of row j) and the row
    // sum, both in the frame of the latest used block max f.
    f32x16_t acc[NM];
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[mt][e] = 0.f;
    float l_run = 0.f;
    float m_run = kNegClamp, f_run = kNegClamp;
    constexpr float kLog2e = 1.4426950408889634f;
    const bf16x2_t ones2 = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);

    // per-lane LDS byte offsets within a block buffer: K operand token j, dims
    // 8h..; V^T operand (16-lane group g: dims 16(g&1)..+15, tokens 4h..4h+3,
    // lane pc addressing token 4h + pc/4, dims 4(pc%4)..+3)
    const uint32_t kofs = j * RB + 16 * h;
    const int g = lane >> 4, pc = lane & 15;
    const uint32_t vofs = (4 * h + (pc >> 2)) * RB + 32 * (g & 1) + 8 * (pc & 3);

    // The value of the other lane half (lane l ^ 32), combined with this
    // lane's: both halves get the same result (lower half's operand first).
    auto halves_max = [](float x) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    };
    auto halves_sum = [](float x) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    };

    // Scheduling: LDS reads are issued ahead of the MFMAs that consume them
    // (an LDS read takes longer than one stage of MFMAs), and the group
    // barriers pin the order of reads, VALU work and MFMAs in a stage.
    constexpr int kDsRead = 0x100, kValu = 0x002, kMfma = 0x008;
    constexpr int KA = 1;  // QK stages (k-steps) the K reads run ahead
    constexpr int VA = 2;  // PV stages (single MFMAs) the V^T reads run ahead
    constexpr int NPV = NM * PS;  // PV stages
    static_assert(NM % 2 == 0, "PV runs over pairs of O^T tiles");
    // next: the fill of the next block (its loads spread over the QK stages).
    auto compute = [&](const char *kb, int blk, bool blk_bad, const Fill &next) {
        const bool first = (blk == blk_begin);
        uint32_t fbase, fcc;
        fill_regs(fbase, fcc);
        // ---- QK: stage = one 16-dim k-step over the NT token tiles ----
        f32x16_t s[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) s[t][e] = 0.f;
        u32x4_t kf[KA + 1][NT];
        auto load_k = [&](int kk, u32x4_t (&dst)[NT]) {
#pragma unroll
            for (int t = 0; t < NT; ++t) dst[t] = lds_ld16(kb, kofs + t * 32 * RB + 32 * kk);
        };
#pragma unroll
        for (int kk = 0; kk < KA; ++kk) load_k(kk, kf[kk]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
            for (int ii = 0; ii < NII; ++ii)
                if (ii * KS / NII == kk) fill_one(next, ii, fbase, fcc);
            if (kk + KA < KS) load_k(kk + KA, kf[(kk + KA) % (KA + 1)]);
#pragma unroll
            for (int t = 0; t < NT; ++t) s[t] = mma_32x32x16(kf[kk % (KA + 1)][t], qv[kk], s[t]);
            if (kk + KA < KS) __builtin_amdgcn_sched_group_barrier(kDsRead, NT, 0);
            __builtin_amdgcn_sched_group_barrier(kMfma, NT, 0);
            __builtin_amdgcn_sched_barrier(0);
        }

        // ---- V^T operand reads of the first PV stages go out before the
        // softmax math (they do not depend on it). Stage q = (pair q / (2 PS),
        // k-step (q / 2) % PS, tile 2 (q / (2 PS)) + q % 2) ----
        i16x4_t vf[VA + 1][2];
        auto stage_tile = [](int q) { return 2 * (q / (2 * PS)) + (q & 1); };
        auto stage_kstep = [](int q) { return (q >> 1) % PS; };
        auto load_v = [&](int q, i16x4_t (&dst)[2]) {
            const uint32_t o = vofs + 64 * stage_tile(q) + 16 * stage_kstep(q) * RB;
            dst[0] = lds_ld_tr(kb, o);
            dst[1] = lds_ld_tr(kb, o + 8 * RB);
        };
#pragma unroll
        for (int q = 0; q < VA; ++q) load_v(q, vf[q]);
        __builtin_amdgcn_sched_barrier(0);

        // ---- mask, block max of s*scale (golden :145-165). For scale > 0 the
        // max of the scaled scores is the scaled max; otherwise scale first ----
        float sc = P.scale;
        if (!(sc > 0.f)) {
#pragma unroll
            for (int t = 0; t < NT; ++t) s[t] *= sc;
            sc = 1.f;
        }
        const int blk0 = blk * BS;
        const bool full = !blk_bad && (blk0 + BS <= min_rowlen);
        if (!full) {
            const int rvalid = blk_bad ? 0 : rowlen - blk0;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (32 * t + 8 * (e >> 2) + 4 * h + (e & 3) >= rvalid) s[t][e] = -INFINITY;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[t][e]);
        mx = halves_max(mx);
        const float mb = fmaxf(mx * sc, kNegClamp);
        // ---- online merge (aiv_online_update.cpp:183-207) in the block frame ----
        const float mnew = first ? mb : fmaxf(m_run, mb);
        const bool use = first || (mb >= mnew - kFrameGap);
        const float cf = first ? 0.f : (use ? __expf(f_run - mb) : 1.f);
        // ---- p = bf16(exp(s*scale - m_blk)) = bf16(exp2(s*scale*log2e - m_blk*log2e)) ----
        const float mb2 = use ? mb * kLog2e : INFINITY;  // a skipped block gives p = 0
        const float sc2 = sc * kLog2e;
        u32x4_t pk[PS];
        float lsum = 0.f;
#pragma unroll
        for (int ks = 0; ks < PS; ++ks) {
            const int t = ks >> 1, s8 = 8 * (ks & 1);
            unsigned w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][s8 + 2 * i], sc2, -mb2));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][s8 + 2 * i + 1], sc2, -mb2));
                w[i] = pack_bf16x2(p0, p1);
                lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[i]), ones2, lsum, false);
            }
            pk[ks] = (u32x4_t){w[0], w[1], w[2], w[3]};
        }
        lsum = halves_sum(lsum);  // the row's other 32 tokens
        m_run = mnew;
        if (use) f_run = mb;
        l_run = l_run * cf + lsum;
        acc[0] *= cf;
        acc[1] *= cf;
        __builtin_amdgcn_sched_barrier(0);

        // ---- A' = e^{f - m_blk} A + P V over pairs of O^T tiles: a pair's
        // MFMAs alternate between its two tiles (an MFMA right after one into
        // the same accumulator waits for it), and the next pair is rescaled
        // during them ----
        constexpr int RPS = 32 / (2 * PS);  // rescale multiplies per stage
#pragma unroll
        for (int q = 0; q < NPV; ++q) {
            const int mt = stage_tile(q), ks = stage_kstep(q);
            const int pair = q / (2 * PS), qi = q % (2 * PS);
            if (q + VA < NPV) load_v(q + VA, vf[(q + VA) % (VA + 1)]);
            if (2 * pair + 2 < NM) {
#pragma unroll
                for (int e = 0; e < RPS; ++e) {
                    const int idx = qi * RPS + e;  // of the next pair's 32 values
                    acc[2 * pair + 2 + idx / 16][idx % 16] *= cf;
                }
            }
            const i16x4_t *vv = vf[q % (VA + 1)];
            const u32x4_t va = __builtin_bit_cast(u32x4_t, __builtin_shufflevector(vv[0], vv[1], 0, 1, 2, 3, 4, 5, 6, 7));
            acc[mt] = mma_32x32x16(va, pk[ks], acc[mt]);
            if (q + VA < NPV) __builtin_amdgcn_sched_group_barrier(kDsRead, 2, 0);
            if (2 * pair + 2 < NM) __builtin_amdgcn_sched_group_barrier(kValu, RPS, 0);
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // ---- block loop: wait + barrier, then the math on this block with the
    // next block's fill spread over it (as loads of nothing where there is no
    // such block) ----
    // Vector memory ops complete in order. Before the loop, one wait for
    // everything: the Q rows and the first block's fill. It is unconditional
    // so that the compiler knows those loads are complete and inserts no
    // waits for them inside the loop (a wait there would also wait for the
    // next block's fill, which it does not count). At the top of iteration
    // blk > blk_begin this wave's only outstanding loads are the fill of blk:
    // the wait for all of them completes it. lgkmcnt(0): this wave's LDS
    // reads of the buffer about to be refilled are done.
    // (A second stream that touched every 128-byte line of the block two
    // ahead, so that its fill hit L2, made cfg4 2.5% slower and the 32-token
    // block shape 7% slower, with one shape of 32 query rows 3% faster.)
    // s_waitcnt immediate: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
    constexpr unsigned kWaitAll = 0x0070u;  // vmcnt(0) expcnt(7) lgkmcnt(0)
    bool bad_cur = false, any_bad = false;
    {
        const Fill f0 = fill_of(blk_begin, smem0, bad_cur);
        uint32_t fbase, fcc;
        fill_regs(fbase, fcc);
#pragma unroll
        for (int ii = 0; ii < NII; ++ii) fill_one(f0, ii, fbase, fcc);
        __builtin_amdgcn_s_waitcnt(kWaitAll);
    }
    for (int blk = blk_begin; blk < blk_end; ++blk) {
        const bool even = ((blk - blk_begin) & 1) == 0;
        __builtin_amdgcn_sched_barrier(0);
        if (blk > blk_begin) __builtin_amdgcn_s_waitcnt(kWaitAll);
        __builtin_amdgcn_s_barrier();  // every wave's fill landed; the other buffer is free
        __builtin_amdgcn_sched_barrier(0);
        bool bad_next = false;
        // the buffer not read by this block takes the next one (or zeros)
        const Fill next = fill_of(blk + 1 < blk_end ? blk + 1 : -1, even ? smem1 : smem0, bad_next);
        any_bad |= bad_cur;
        if (active) {
            compute(even ? smem0 : smem1, blk, bad_cur, next);
        } else {  // no rows: the loads only
            uint32_t fbase, fcc;
            fill_regs(fbase, fcc);
#pragma unroll
            for (int ii = 0; ii < NII; ++ii) fill_one(next, ii, fbase, fcc);
        }
        bad_cur = bad_next;
    }
    __builtin_amdgcn_s_waitcnt(kWaitAll);  // the last zero fill is done before the next segment's
    if (any_bad && threadIdx.x == 0) atomicOr(P.error_flag, kErrBadBlock);
    __syncthreads();  // the buffers are refilled by the next segment

    // ---- finish: O = e^{f-m} A, l = e^{f-m} L; lane (h, j) holds dims
    // 32mt + 8a + 4h + e (register 4a+e of tile mt) of row j ----
    if (!active || j >= rows_here) return;
    const int row = r0 + j;
    if (blk_begin == 0 && blk_end == nblk) {  // the whole tile: final output
        const float inv = l_run > 0.f ? 1.f / l_run : 0.f;  // the frame factor cancels
        const int64_t off = out_row_offset(P, b, kvh, row, DV) + 4 * h;
#pragma unroll
        for (int mt = 0; mt < NM; ++mt)
#pragma unroll
            for (int a = 0; a < 4; ++a)
                OutStore<OutT>::store4(
                    P.out, off + 32 * mt + 8 * a,
                    (f32x4_t){acc[mt][4 * a], acc[mt][4 * a + 1], acc[mt][4 * a + 2], acc[mt][4 * a + 3]} * inv);
        return;
    }
    // ---- a piece of the tile: partial (O relative to m, plus m and l) per
    // 16-row tile (the merge kernel's unit) ----
    const float osc = __expf(f_run - m_run);
    const int64_t piece = ((int64_t)slice * P.tiles_per_worker + (row >> 4)) * 2 + slot;
    float *dst = P.part_o + (piece * 16 + (row & 15)) * DV + 4 * h;
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
        for (int a = 0; a < 4; ++a)
            *reinterpret_cast<f32x4_t *>(dst + 32 * mt + 8 * a) =
                (f32x4_t){acc[mt][4 * a], acc[mt][4 * a + 1], acc[mt][4 * a + 2], acc[mt][4 * a + 3]} * osc;
    if (h == 0) {
        P.part_ml[piece * 32 + (row & 15)] = m_run;
        P.part_ml[piece * 32 + 16 + (row & 15)] = l_run * osc;
    }
}

// Worker workgroup = four waves = one row group (up to 128 query rows) of one
// work slice. The work list holds (batch, kv head, KV block) entries; every
// row group of a slice walks the same entries.
template <int BS, int DK, int DV, typename OutT>
__global__ void __launch_bounds__(256) pa_mla_kernel(const KernelParams P) {
    using L = MlaLayout<DK>;
    __shared__ __attribute__((aligned(16))) char smem0[BS * L::kRowBytes];
    __shared__ __attribute__((aligned(16))) char smem1[BS * L::kRowBytes];
    flag_bad_lengths(P);
    const int groups = (P.rows + kMlaRowsPerGroup - 1) / kMlaRowsPerGroup;
    int slice = 0, rgrp = 0;
    mla_worker(blockIdx.x, P.workers, groups, &slice, &rgrp);
    const int tpb = P.kv_heads;  // work-list tiles per batch
    int start = 0, end = 0, b = 0, prefix = 0, ctx0 = 0;
    locate_slice(P, slice, &start, &end, &b, &prefix, &ctx0);  // identical in every wave
    // wave-uniform values, kept in scalar registers
    start = __builtin_amdgcn_readfirstlane(start);
    end = __builtin_amdgcn_readfirstlane(end);
    b = __builtin_amdgcn_readfirstlane(b);
    prefix = __builtin_amdgcn_readfirstlane(prefix);
    if (start >= end) return;
    int nb = (__builtin_amdgcn_readfirstlane(ctx0) + BS - 1) / BS;
    if (nb == 0) return;
    // Work units: each (batch, kv head) tile takes seg_cost units, then one
    // per block. The slice [start, end) runs the blocks whose units it holds.
    const int span = nb + P.seg_cost;
    int kvh = (start - prefix) / span;
    int t0 = prefix + kvh * span;  // the tile's first unit
    int slot = 0;
    while (nb > 0) {
        const int blk0 = max(0, start - t0 - P.seg_cost), blk1 = min(nb, end - t0 - P.seg_cost);
        if (blk1 > blk0) {
            run_mla_segment<BS, DK, DV, OutT>(P, slice, rgrp, b, kvh, nb, blk0, blk1, slot, smem0, smem1);
            slot = 1;
        }
        t0 += nb + P.seg_cost;
        if (t0 >= end) break;
        if (++kvh == tpb) {
            kvh = 0;
            do {
                ++b;
                nb = blocks_of(P, b);
            } while (nb == 0 && b + 1 < P.batch);
            if (nb == 0) break;
        }
    }
}


// ---------------------------------------------------------------------------
// Kernel sets. Each set is instantiated in its own translation unit
// (pa_kernels_*.hip); the host side picks kernels through these functions.
// ---------------------------------------------------------------------------

typedef void (*KernelFn)(KernelParams);

constexpr int kMlaDk = 576, kMlaDv = 512;

struct KernelPair {
    KernelFn main;        // one wave per worker (MLA: the four-wave LDS kernel); null if unsupported
    KernelFn main_multi;  // up to kMaxWavesPerWorker waves per worker
    bool mla;
    bool klds;  // stages K through LDS (full-row K reads); main_multi in dynamic LDS, BS x 256 B per wave
    KernelFn main_pair = nullptr;  // one wave per worker running two row tiles (K through LDS), or null
};

struct MergeFn {
    KernelFn fn;  // null if unsupported
    int threads;  // workgroup size
};

// GQA decode with 16-bit query and caches of element type `dt` (the
// SIMPLER_HIP_DT_BFLOAT16 or SIMPLER_HIP_DT_FLOAT16 code), Dk == Dv.
KernelPair pick_gqa_bf16(int bs, int d, int out_dtype);
KernelPair pick_gqa_f16(int bs, int d, int out_dtype);
// The same with the fused KV append (KernelParams::k_new / v_new).
KernelPair pick_gqa_bf16_append(int bs, int d, int out_dtype);
KernelPair pick_gqa_f16_append(int bs, int d, int out_dtype);
// GQA decode with fp8 E4M3FN caches (bf16 query), Dk == Dv == 128.
KernelPair pick_gqa_fp8(int bs, int d, int out_dtype);
// MLA (Dk 576, Dv 512, V a prefix of K), bf16.
KernelPair pick_mla(int bs, int out_dtype);
// The split merge for output width dv.
MergeFn pick_merge(int dv, int out_dtype);

}  // namespace pa
}  // namespace simpler_hip
