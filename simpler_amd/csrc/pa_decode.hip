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
//  kernels/kernel/pa_kernel.cce:1634-1773), done in-kernel by the last split
// of each (batch, kv head, row tile) to finish.
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
// Work decomposition: one 64-lane wavefront per (split, kv head, row tile,
// batch). A row is one (query token, head in the GQA group) pair; 16 rows per
// tile (MFMA N). A split is a contiguous run of KV blocks of one sequence.
// Lane (qd = lane/16, pc = lane%16):
//   QK   A operand = K token pc of the tile, dims 32kk+8qd..+7 (one 16-B load)
//        B operand = Q row pc, same dims
//        C         = S[row pc][tokens 4qd..4qd+3]   (S^T tile)
//   PV   A operand = P[row pc][tokens 4qd..4qd+3]  == the QK C layout (no shuffle)
//        B operand = V[tokens 4qd..4qd+3][dim 8pc+jj], built from four 16-B row
//                    loads by an in-register 4x8 bf16 transpose
//        C         = O[rows 4qd..4qd+3][dim 8pc+jj]
// K of the next block is prefetched while the current block's softmax and PV
// run; V of a block is issued before its QK.

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "simpler_hip/pa_decode.h"

namespace simpler_hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

constexpr float kNegClamp = -1e30f;  // goldens/paged_attention.py:160 clamp
constexpr float kFrameGap = 40.f;
constexpr int kMaxBlocksPerSplit = 64;  // one block-table entry per lane
constexpr int kMaxSplits = 64;
// The split counters live in a fixed region at the start of every workspace,
// sized for kCounterCapacity tiles whatever the plan: partial results of one
// plan must never land where another plan's counters are, because the
// counters rely on being zero between launches.
constexpr int64_t kCounterCapacity = 65536;
#ifndef SIMPLER_HIP_PREFETCH_K
#define SIMPLER_HIP_PREFETCH_K 0
#endif
// 1: K of block i+1 is loaded while block i's softmax and PV run (costs a
//    second block of K registers); 0: K and V of a block are both issued at
//    the top of its iteration.
constexpr bool kPrefetchK = SIMPLER_HIP_PREFETCH_K != 0;

struct KernelParams {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    const int32_t *block_table;
    const int32_t *context_lens;
    void *out;
    float *part_o;       // [n_tiles][max_splits][16][DV]
    float *part_ml;      // [n_tiles][max_splits][2][16]  (m row values, then l)
    unsigned *counters;  // [n_tiles], zero between launches
    unsigned *error_flag;
    int64_t k_block_stride, k_token_stride, k_head_stride;
    int64_t v_block_stride, v_token_stride, v_head_stride;
    int32_t batch, q_len, num_heads, kv_heads, group, rows, row_tiles;
    int32_t max_blocks, num_pool_blocks;
    int32_t blocks_per_split, max_splits;
    float scale;
    int32_t causal;
};

__device__ __forceinline__ u32x4_t ld16(const uint16_t *p) { return *reinterpret_cast<const u32x4_t *>(p); }

__device__ __forceinline__ unsigned pack_bf16x2(float a, float b) {
    // fp32 -> bf16 round-to-nearest-even (gfx950: v_cvt_pk_bf16_f32)
    const bf16x2_t h = __builtin_convertvector((f32x2_t){a, b}, bf16x2_t);
    return __builtin_bit_cast(unsigned, h);
}

__device__ __forceinline__ float bf16lo_to_f32(unsigned w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi_to_f32(unsigned w) { return __uint_as_float(w & 0xffff0000u); }

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

// Output element offset of (row r of kv head kvh, dim 0).
__device__ __forceinline__ int64_t out_row_offset(const KernelParams &P, int b, int kvh, int r, int dv) {
    const int i = r / P.group, hh = r - i * P.group;
    return ((int64_t)(b * P.q_len + i) * P.num_heads + kvh * P.group + hh) * dv;
}

template <int BS, int DK, int DV, typename OutT>
__global__ void __launch_bounds__(64) pa_decode_splitk_kernel(const KernelParams P) {
    static_assert(BS % 16 == 0 && BS >= 16 && BS <= 128, "block_size must be 16..128, multiple of 16");
    static_assert(DK % 8 == 0 && DV % 8 == 0, "head dims must be multiples of 8");
    constexpr int NT = BS / 16;           // 16-token tiles per KV block
    constexpr int KS = (DK + 31) / 32;    // 32-dim k-steps of QK
    constexpr int DVS = (DV + 127) / 128; // 128-dim column sets of PV

    const int lane = threadIdx.x;
    const int qd = lane >> 4;
    const int pc = lane & 15;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y / P.row_tiles;
    const int rt = blockIdx.y - kvh * P.row_tiles;
    const int b = blockIdx.z;
    const int tile_id = (b * P.kv_heads + kvh) * P.row_tiles + rt;

    int ctx = P.context_lens[b];
    ctx = min(max(ctx, 0), P.max_blocks * BS);
    const int nblk = (ctx + BS - 1) / BS;
    const int bps = P.blocks_per_split;
    const int nsplit = (nblk + bps - 1) / bps;
    if (split >= (nsplit > 0 ? nsplit : 1)) return;

    const int rows_here = min(16, P.rows - rt * 16);

    if (nblk == 0) {  // empty context: defined as a zero output
        for (int idx = lane; idx < rows_here * (DV / 4); idx += 64) {
            const int row = idx / (DV / 4), c4 = idx - row * (DV / 4);
            OutStore<OutT>::store4(P.out, out_row_offset(P, b, kvh, rt * 16 + row, DV) + 4 * c4,
                                   (f32x4_t){0.f, 0.f, 0.f, 0.f});
        }
        return;
    }

    // ---- Q^T operand (row pc, dims 32kk+8qd..) and this row's visible length ----
    int rowlen = 0;
    u32x4_t qv[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qv[kk] = (u32x4_t){0u, 0u, 0u, 0u};
    if (pc < rows_here) {
        const int r = rt * 16 + pc;
        const int i = r / P.group, hh = r - i * P.group;
        const uint16_t *qrow = P.q + ((int64_t)(b * P.q_len + i) * P.num_heads + kvh * P.group + hh) * DK + 8 * qd;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            if (DK % 32 == 0 || 32 * kk + 8 * qd < DK) qv[kk] = ld16(qrow + 32 * kk);
        }
        rowlen = P.causal ? ctx - (P.q_len - 1 - i) : ctx;
    }
    // shortest visible length over the valid rows of this tile (wave-uniform):
    // blocks that end at or before it need no masking.
    const int min_rowlen = P.causal ? ctx - (P.q_len - 1 - (rt * 16) / P.group) : ctx;

    const int blk_begin = split * bps;
    const int blk_end = min(nblk, blk_begin + bps);

    // Block-table entries of this split, one per lane.
    const int32_t *bt_row = P.block_table + (int64_t)b * P.max_blocks;
    const int bt_val = (blk_begin + lane < blk_end) ? bt_row[blk_begin + lane] : 0;

    f32x4_t acc[DVS][8];
#pragma unroll
    for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) acc[ds][jj] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    float m_run = kNegClamp, f_run = kNegClamp, l_part = 0.f;

    u32x4_t kreg[NT][KS];
    u32x4_t vreg[NT][DVS][4];

    const uint16_t *kbase_h = P.k + (int64_t)kvh * P.k_head_stride + 8 * qd;
    const uint16_t *vbase_h = P.v + (int64_t)kvh * P.v_head_stride + 8 * pc;

    auto phys_of = [&](int blk, bool &bad) -> int {
        const int phys = __builtin_amdgcn_readlane(bt_val, blk - blk_begin);
        bad = (unsigned)phys >= (unsigned)P.num_pool_blocks;
        return bad ? 0 : phys;
    };
    auto load_k = [&](int phys) {
        const uint16_t *kb = kbase_h + (int64_t)phys * P.k_block_stride;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint16_t *kt = kb + (int64_t)(16 * t + pc) * P.k_token_stride;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                if (DK % 32 == 0 || 32 * kk + 8 * qd < DK)
                    kreg[t][kk] = ld16(kt + 32 * kk);
                else
                    kreg[t][kk] = (u32x4_t){0u, 0u, 0u, 0u};
            }
        }
    };
    auto load_v = [&](int phys) {
        const uint16_t *vb = vbase_h + (int64_t)phys * P.v_block_stride;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint16_t *vt = vb + (int64_t)(16 * t + 4 * qd + e) * P.v_token_stride;
#pragma unroll
                for (int ds = 0; ds < DVS; ++ds) {
                    if (DV % 128 == 0 || 128 * ds + 8 * pc < DV)
                        vreg[t][ds][e] = ld16(vt + 128 * ds);
                    else
                        vreg[t][ds][e] = (u32x4_t){0u, 0u, 0u, 0u};
                }
            }
    };

    bool bad = false;
    int phys = phys_of(blk_begin, bad);
    if (kPrefetchK) load_k(phys);

    for (int blk = blk_begin; blk < blk_end; ++blk) {
        const bool first = (blk == blk_begin);
        if (blk != blk_begin && !kPrefetchK) phys = phys_of(blk, bad);
        if (bad && lane == 0) atomicOr(P.error_flag, 1u);
        if (!kPrefetchK) load_k(phys);
        load_v(phys);

        // ---- QK: S^T tiles ----
        f32x4_t s[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            f32x4_t c = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kreg[t][kk]),
                                                            __builtin_bit_cast(bf16x8_t, qv[kk]), c, 0, 0, 0);
            s[t] = c;
        }

        // ---- prefetch K of the next block ----
        const bool blk_bad = bad;
        if (kPrefetchK && blk + 1 < blk_end) {
            phys = phys_of(blk + 1, bad);
            load_k(phys);
        }

        // ---- softmax prepare: mask, scale, block max (golden :145-165) ----
        const int blk0 = blk * BS;
        const bool full = !blk_bad && (blk0 + BS <= min_rowlen);
        const int rvalid = blk_bad ? 0 : rowlen - blk0;  // tokens of this block visible to row pc
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float x = s[t][e] * P.scale;
                if (!full) x = (16 * t + 4 * qd + e < rvalid) ? x : -INFINITY;
                s[t][e] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mb = fmaxf(mx, kNegClamp);

        // ---- online merge coefficients (aiv_online_update.cpp:183-207) ----
        const float mnew = first ? mb : fmaxf(m_run, mb);
        const bool use = first || (mb >= mnew - kFrameGap);
        const float alpha = first ? 0.f : __expf(m_run - mnew);
        const float beta = __expf(mb - mnew);
        const float cf = first ? 0.f : (use ? __expf(f_run - mb) : 1.f);

        // ---- p = bf16(exp(s - m_blk)); l_blk = sum of the rounded p ----
        i16x4_t pa[NT];
        float lb = 0.f;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float p[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) p[e] = use ? __expf(s[t][e] - mb) : 0.f;
            const unsigned w0 = pack_bf16x2(p[0], p[1]);
            const unsigned w1 = pack_bf16x2(p[2], p[3]);
            lb += (bf16lo_to_f32(w0) + bf16hi_to_f32(w0)) + (bf16lo_to_f32(w1) + bf16hi_to_f32(w1));
            pa[t] = __builtin_bit_cast(i16x4_t, (u32x2_t){w0, w1});
        }
        l_part = first ? lb : alpha * l_part + beta * lb;
        m_run = mnew;
        if (use) f_run = mb;

        // ---- rescale A to the new frame (rows 4qd+e live in lane 4qd+e's cf) ----
        {
            f32x4_t cv;
#pragma unroll
            for (int e = 0; e < 4; ++e) cv[e] = __shfl(cf, 4 * qd + e, 64);
#pragma unroll
            for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) acc[ds][jj] *= cv;
        }

        // ---- PV: A += P * V ----
        const int vvalid = blk_bad ? 0 : min(BS, ctx - blk0);  // tokens with defined V
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (vvalid < BS) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (16 * t + 4 * qd + e >= vvalid)
#pragma unroll
                        for (int ds = 0; ds < DVS; ++ds) vreg[t][ds][e] = (u32x4_t){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int ds = 0; ds < DVS; ++ds)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int w = jj >> 1;
                    const unsigned a0 = vreg[t][ds][0][w], a1 = vreg[t][ds][1][w];
                    const unsigned a2 = vreg[t][ds][2][w], a3 = vreg[t][ds][3][w];
                    unsigned d0, d1;
                    if (jj & 1) {
                        d0 = (a0 >> 16) | (a1 & 0xffff0000u);
                        d1 = (a2 >> 16) | (a3 & 0xffff0000u);
                    } else {
                        d0 = (a0 & 0xffffu) | (a1 << 16);
                        d1 = (a2 & 0xffffu) | (a3 << 16);
                    }
                    acc[ds][jj] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        pa[t], __builtin_bit_cast(i16x4_t, (u32x2_t){d0, d1}), acc[ds][jj], 0, 0, 0);
                }
        }
    }

    // ---- finish this split: O = e^{f-m} A, l = sum over the four lane groups ----
    float l_tot = l_part + __shfl_xor(l_part, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
    const float osc = __expf(f_run - m_run);
    float l_e[4], o_e[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        l_e[e] = __shfl(l_tot, 4 * qd + e, 64);
        o_e[e] = __shfl(osc, 4 * qd + e, 64);
    }

    if (nsplit == 1) {
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

    // ---- write this split's partial (O relative to m, plus m and l) ----
    float *po = P.part_o + ((int64_t)tile_id * P.max_splits + split) * 16 * DV;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int row = 4 * qd + e;
        if (row >= rows_here) continue;
#pragma unroll
        for (int ds = 0; ds < DVS; ++ds) {
            if (!(DV % 128 == 0 || 128 * ds + 8 * pc < DV)) continue;
            float *dst = po + row * DV + 128 * ds + 8 * pc;
            *reinterpret_cast<f32x4_t *>(dst) =
                (f32x4_t){acc[ds][0][e], acc[ds][1][e], acc[ds][2][e], acc[ds][3][e]} * o_e[e];
            *reinterpret_cast<f32x4_t *>(dst + 4) =
                (f32x4_t){acc[ds][4][e], acc[ds][5][e], acc[ds][6][e], acc[ds][7][e]} * o_e[e];
        }
    }
    float *pml = P.part_ml + ((int64_t)tile_id * P.max_splits + split) * 32;
    if (qd == 0) {
        pml[pc] = m_run;
        pml[16 + pc] = l_tot;
    }
    __threadfence();
    unsigned prev = 0;
    if (lane == 0) prev = atomicAdd(&P.counters[tile_id], 1u);
    prev = __shfl(prev, 0, 64);
    if (prev != (unsigned)(nsplit - 1)) return;
    __threadfence();

    // ---- last split of this tile: log-sum-exp merge over the splits ----
    const float *ml = P.part_ml + (int64_t)tile_id * P.max_splits * 32;
    const float *pob = P.part_o + (int64_t)tile_id * P.max_splits * 16 * DV;
    for (int idx = lane; idx < rows_here * (DV / 4); idx += 64) {
        const int row = idx / (DV / 4), c4 = idx - row * (DV / 4);
        float M = -INFINITY;
        for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, ml[sp * 32 + row]);
        float L = 0.f;
        f32x4_t o = (f32x4_t){0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < nsplit; ++sp) {
            const float w = __expf(ml[sp * 32 + row] - M);
            L += w * ml[sp * 32 + 16 + row];
            o += w * *reinterpret_cast<const f32x4_t *>(pob + ((int64_t)sp * 16 + row) * DV + 4 * c4);
        }
        const f32x4_t res = L > 0.f ? o / L : (f32x4_t){0.f, 0.f, 0.f, 0.f};
        OutStore<OutT>::store4(P.out, out_row_offset(P, b, kvh, rt * 16 + row, DV) + 4 * c4, res);
    }
    if (lane == 0) atomicExch(&P.counters[tile_id], 0u);
}

// ----------------------------------------------------------------------------
// Host side: validation, split plan, dispatch
// ----------------------------------------------------------------------------

struct Plan {
    int bps;
    int max_splits;
    int row_tiles;
    int rows;
    size_t part_o_bytes, part_ml_bytes, counter_bytes;
    size_t total;
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int validate(const SimplerHipPaDecodeArgs *a) {
    if (!a) return SIMPLER_HIP_ERR_INVALID;
    if (!a->query || !a->key_cache || !a->value_cache || !a->block_table || !a->context_lens || !a->out)
        return SIMPLER_HIP_ERR_INVALID;
    if (a->batch < 0 || a->q_len < 1 || a->num_kv_heads < 1 || a->num_heads < 1) return SIMPLER_HIP_ERR_INVALID;
    if (a->num_heads % a->num_kv_heads) return SIMPLER_HIP_ERR_INVALID;
    if (a->head_dim_k < 8 || a->head_dim_v < 8 || a->head_dim_k % 8 || a->head_dim_v % 8)
        return SIMPLER_HIP_ERR_INVALID;
    if (a->block_size < 1 || a->max_blocks_per_seq < 1 || a->num_blocks < 1) return SIMPLER_HIP_ERR_INVALID;
    const int64_t strides[6] = {a->k_block_stride, a->k_token_stride, a->k_head_stride,
                                a->v_block_stride, a->v_token_stride, a->v_head_stride};
    for (int64_t s : strides)
        if (s <= 0 || s % 8) return SIMPLER_HIP_ERR_INVALID;  // 16-byte aligned rows
    if (a->out_dtype != SIMPLER_HIP_DT_FLOAT32 && a->out_dtype != SIMPLER_HIP_DT_BFLOAT16)
        return SIMPLER_HIP_ERR_UNSUPPORTED;
    if (!(a->scale == a->scale)) return SIMPLER_HIP_ERR_INVALID;
    if (a->blocks_per_split < 0 || a->blocks_per_split > kMaxBlocksPerSplit) return SIMPLER_HIP_ERR_INVALID;
    {
        const int group = a->num_heads / a->num_kv_heads;
        const int64_t row_tiles = ((int64_t)group * a->q_len + 15) / 16;
        if ((int64_t)a->batch * a->num_kv_heads * row_tiles > kCounterCapacity) return SIMPLER_HIP_ERR_UNSUPPORTED;
    }
    if (((uintptr_t)a->query | (uintptr_t)a->key_cache | (uintptr_t)a->value_cache | (uintptr_t)a->out) & 15)
        return SIMPLER_HIP_ERR_INVALID;
    return SIMPLER_HIP_OK;
}

Plan make_plan(const SimplerHipPaDecodeArgs *a) {
    Plan p{};
    const int group = a->num_heads / a->num_kv_heads;
    p.rows = group * a->q_len;
    p.row_tiles = (p.rows + 15) / 16;
    const int64_t n_tiles = (int64_t)a->batch * a->num_kv_heads * p.row_tiles;
    int bps = a->blocks_per_split;
    if (bps <= 0) {
        // Aim for ~4 KV blocks per wavefront when there is enough work to
        // fill the chip several times over, and never more than kMaxSplits
        // splits per tile (bounds the in-kernel merge).
        const int64_t target_waves = 4096;
        int64_t work = n_tiles * a->max_blocks_per_seq;
        int64_t b = (work + target_waves - 1) / target_waves;
        if (b < 4) b = 4;
        const int64_t min_for_cap = (a->max_blocks_per_seq + kMaxSplits - 1) / kMaxSplits;
        if (b < min_for_cap) b = min_for_cap;
        if (b > kMaxBlocksPerSplit) b = kMaxBlocksPerSplit;
        bps = (int)b;
    }
    p.bps = bps;
    p.max_splits = (a->max_blocks_per_seq + bps - 1) / bps;
    const int dv = a->head_dim_v;
    // Layout: [error word | counters, fixed capacity] [m,l partials] [O partials]
    p.counter_bytes = align_up((size_t)(kCounterCapacity + 1) * sizeof(unsigned), 256);
    p.part_ml_bytes = align_up((size_t)n_tiles * p.max_splits * 32 * sizeof(float), 256);
    p.part_o_bytes = align_up((size_t)n_tiles * p.max_splits * 16 * dv * sizeof(float), 256);
    p.total = p.counter_bytes + p.part_ml_bytes + p.part_o_bytes;
    return p;
}

typedef void (*KernelFn)(KernelParams);

template <int BS, int D, typename OutT>
KernelFn pick_fn() {
    return pa_decode_splitk_kernel<BS, D, D, OutT>;
}

template <int BS, typename OutT>
KernelFn pick_d(int dk, int dv) {
    if (dk != dv) return nullptr;
    switch (dk) {
        case 16: return pick_fn<BS, 16, OutT>();
        case 32: return pick_fn<BS, 32, OutT>();
        case 64: return pick_fn<BS, 64, OutT>();
        case 128: return pick_fn<BS, 128, OutT>();
        case 256:
            if constexpr (BS <= 64) return pick_fn<BS, 256, OutT>();
            return nullptr;
        default: return nullptr;
    }
}

template <typename OutT>
KernelFn pick_bs(int bs, int dk, int dv) {
    switch (bs) {
        case 16: return pick_d<16, OutT>(dk, dv);
        case 32: return pick_d<32, OutT>(dk, dv);
        case 64: return pick_d<64, OutT>(dk, dv);
        case 128: return pick_d<128, OutT>(dk, dv);
        default: return nullptr;
    }
}

KernelFn pick_kernel(const SimplerHipPaDecodeArgs *a) {
    if (a->out_dtype == SIMPLER_HIP_DT_FLOAT32) return pick_bs<float>(a->block_size, a->head_dim_k, a->head_dim_v);
    if (a->out_dtype == SIMPLER_HIP_DT_BFLOAT16) return pick_bs<__bf16>(a->block_size, a->head_dim_k, a->head_dim_v);
    return nullptr;
}

}  // namespace
}  // namespace simpler_hip

using namespace simpler_hip;

extern "C" size_t simpler_hip_pa_decode_workspace_size(const SimplerHipPaDecodeArgs *args) {
    if (validate(args) != SIMPLER_HIP_OK) return 0;
    return make_plan(args).total;
}

extern "C" int simpler_hip_pa_decode_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
    if (!workspace) return SIMPLER_HIP_ERR_WORKSPACE;
    if (hipMemsetAsync(workspace, 0, workspace_bytes, (hipStream_t)stream) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    return SIMPLER_HIP_OK;
}

extern "C" int simpler_hip_pa_decode_plan(const SimplerHipPaDecodeArgs *args, int32_t *blocks_per_split,
                                          int32_t *max_splits) {
    const int rc = validate(args);
    if (rc != SIMPLER_HIP_OK) return rc;
    const Plan p = make_plan(args);
    if (blocks_per_split) *blocks_per_split = p.bps;
    if (max_splits) *max_splits = p.max_splits;
    return SIMPLER_HIP_OK;
}

extern "C" const char *simpler_hip_pa_decode_kernel_name(const SimplerHipPaDecodeArgs *args) {
    if (validate(args) != SIMPLER_HIP_OK || !pick_kernel(args)) return "";
    return "pa_decode_splitk_kernel";
}

extern "C" int simpler_hip_pa_decode(const SimplerHipPaDecodeArgs *a, void *workspace, size_t workspace_bytes,
                                     void *stream) {
    int rc = validate(a);
    if (rc != SIMPLER_HIP_OK) return rc;
    KernelFn fn = pick_kernel(a);
    if (!fn) return SIMPLER_HIP_ERR_UNSUPPORTED;
    const Plan plan = make_plan(a);
    if (!workspace || workspace_bytes < plan.total || ((uintptr_t)workspace & 255)) return SIMPLER_HIP_ERR_WORKSPACE;
    if (a->batch == 0) return SIMPLER_HIP_OK;

    KernelParams P{};
    P.q = (const uint16_t *)a->query;
    P.k = (const uint16_t *)a->key_cache;
    P.v = (const uint16_t *)a->value_cache;
    P.block_table = a->block_table;
    P.context_lens = a->context_lens;
    P.out = a->out;
    char *ws = (char *)workspace;
    P.error_flag = (unsigned *)ws;
    P.counters = (unsigned *)ws + 1;
    P.part_ml = (float *)(ws + plan.counter_bytes);
    P.part_o = (float *)(ws + plan.counter_bytes + plan.part_ml_bytes);
    P.k_block_stride = a->k_block_stride;
    P.k_token_stride = a->k_token_stride;
    P.k_head_stride = a->k_head_stride;
    P.v_block_stride = a->v_block_stride;
    P.v_token_stride = a->v_token_stride;
    P.v_head_stride = a->v_head_stride;
    P.batch = a->batch;
    P.q_len = a->q_len;
    P.num_heads = a->num_heads;
    P.kv_heads = a->num_kv_heads;
    P.group = a->num_heads / a->num_kv_heads;
    P.rows = plan.rows;
    P.row_tiles = plan.row_tiles;
    P.max_blocks = a->max_blocks_per_seq;
    P.num_pool_blocks = a->num_blocks;
    P.blocks_per_split = plan.bps;
    P.max_splits = plan.max_splits;
    P.scale = a->scale;
    P.causal = (a->causal && a->q_len > 1) ? 1 : 0;

    if ((int64_t)a->num_kv_heads * plan.row_tiles > 65535 || a->batch > 65535) return SIMPLER_HIP_ERR_INVALID;
    dim3 grid((unsigned)plan.max_splits, (unsigned)(a->num_kv_heads * plan.row_tiles), (unsigned)a->batch);
    hipLaunchKernelGGL(fn, grid, dim3(64), 0, (hipStream_t)stream, P);
    if (hipGetLastError() != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    return SIMPLER_HIP_OK;
}

extern "C" int simpler_hip_pa_decode_check(void *workspace, size_t workspace_bytes, void *stream) {
    if (!workspace || workspace_bytes < sizeof(unsigned)) return SIMPLER_HIP_ERR_WORKSPACE;
    unsigned flag = 0;
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    if (hipMemcpy(&flag, workspace, sizeof(flag), hipMemcpyDeviceToHost) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    if (flag == 0) return SIMPLER_HIP_OK;
    const unsigned zero = 0;
    if (hipMemcpy(workspace, &zero, sizeof(zero), hipMemcpyHostToDevice) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    return SIMPLER_HIP_ERR_BAD_BLOCK;
}
