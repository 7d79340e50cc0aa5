// Incore kernels of the task-graph backend (gfx950).
//
// One HIP kernel per simpler incore kernel the graph can run. Each restates
// the reference kernel's arithmetic in the reference's order, on ChipTensor
// views (addr + start_offset, row stride = strides[0], unit last-dim stride):
//
//   tg_qk_matmul       <- examples/a2a3/tensormap_and_ringbuffer/paged_attention/kernels/aic/aic_qk_matmul.cpp:38-100
//                         sij = qi * kj^T, bf16 in, fp32 accumulate (MFMA 16x16x32, one wave per 16x16 tile)
//   tg_softmax_prepare <- .../aiv/aiv_softmax_prepare.cpp:96-131
//                         columns >= valid_len -> -inf; s *= scale; m = rowmax; p = exp(s - m);
//                         p rounded to bf16 (RNE); l = rowsum of the rounded p. A row with no
//                         valid column gives m = -1e30, l = 0, p = 0 (the batched variant's rule,
//                         tests/st/a2a3/tensormap_and_ringbuffer/batch_paged_attention/kernels/aiv/
//                         aiv_softmax_prepare.cpp:105-121)
//   tg_pv_matmul       <- .../aic/aic_pv_matmul.cpp:38-99   oi_new = pij * vj (MFMA 16x16x32)
//   tg_online_update   <- .../aiv/aiv_online_update.cpp:125-231
//                         first block: mi = mij, li = lij, oi = oi_new (dst = oi_new / lij if also last);
//                         otherwise m' = max(mi, mij), alpha = exp(mi - m'), beta = exp(mij - m'),
//                         li = alpha*li + beta*lij, oi = alpha*oi + beta*oi_new, dst = oi / li if last
//   tg_vector          <- examples/a2a3/tensormap_and_ringbuffer/vector_example/kernels/aiv/
//                         kernel_add.cpp, kernel_add_scalar.cpp, kernel_mul.cpp (fp32 elementwise)
//
// Every product and sum is rounded on its own (no fused multiply-add), as the
// reference's vector unit does, so results depend only on the operation order
// written here.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "incore.h"
#include "simpler_hip/task_graph.h"

#pragma clang fp contract(off)

namespace simpler_hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));

constexpr float kMaskedRowMax = -1e30f;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((unsigned)b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    const unsigned u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ---------------------------------------------------------------- QK / PV

struct MatParams {
    const uint16_t *a;  // [M, K] rows, unit stride
    const uint16_t *b;  // QK: [N, K] rows (b^T is the operand); PV: [K, N] rows
    float *c;           // [M, N] fp32
    int64_t a_ld, b_ld, c_ld;
    int32_t M, N, K;
};

// 16x16 output tiles, one wave each, four waves per workgroup.
// QK: B operand lane (col j, k-group g) = b[j][k0+8g .. +7] (contiguous).
// PV: B operand lane (col j, k-group g) = b[k0+8g+t][j], t = 0..7 (strided).
template <bool B_ROWS_ARE_COLS>
__global__ void __launch_bounds__(256) tg_matmul_kernel(const MatParams P) {
    const int lane = threadIdx.x & 63;
    const int ntn = (P.N + 15) / 16;
    const int tiles = ((P.M + 15) / 16) * ntn;
    const int tile = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (tile >= tiles) return;
    const int mt = tile / ntn, nt = tile - mt * ntn;
    const int r = lane & 15, g = lane >> 4;
    const int row = mt * 16 + r, col = nt * 16 + r;
    // The operands of KCH k-steps are loaded before their MFMAs, so a wave
    // waits for one memory round trip per 32*KCH of K rather than one per
    // load (K = 128, the tasks' size, is one round trip). K % 8 == 0 (checked
    // at launch), so a lane's 8 k-values are all in range or all out; out of
    // range, the loads read element 0 of the operand (always in bounds) and
    // the value is replaced by zero, with no branch between the loads.
    constexpr int KCH = 4;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    const u32x4_t zero4 = {0u, 0u, 0u, 0u};
    for (int k_base = 0; k_base < P.K; k_base += 32 * KCH) {
        u32x4_t av[KCH], bv[KCH];
#pragma unroll
        for (int c = 0; c < KCH; ++c) {
            const int kk = k_base + 32 * c + 8 * g;
            const bool oka = row < P.M && kk < P.K, okb = col < P.N && kk < P.K;
            const u32x4_t a = *reinterpret_cast<const u32x4_t *>(P.a + (oka ? (int64_t)row * P.a_ld + kk : 0));
            av[c] = oka ? a : zero4;
            if (B_ROWS_ARE_COLS) {
                const u32x4_t b = *reinterpret_cast<const u32x4_t *>(P.b + (okb ? (int64_t)col * P.b_ld + kk : 0));
                bv[c] = okb ? b : zero4;
            } else {
                const int64_t b0 = okb ? (int64_t)kk * P.b_ld + col : 0;
                u16x8_t h;
#pragma unroll
                for (int t = 0; t < 8; ++t) h[t] = P.b[b0 + (int64_t)t * P.b_ld];
                bv[c] = okb ? __builtin_bit_cast(u32x4_t, h) : zero4;
            }
        }
#pragma unroll
        for (int c = 0; c < KCH; ++c)
            if (k_base + 32 * c < P.K)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[c]),
                                                              __builtin_bit_cast(bf16x8_t, bv[c]), acc, 0, 0, 0);
    }
    // C layout: lane holds C[4g + e][r] of the tile.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = mt * 16 + 4 * g + e;
        if (m < P.M && col < P.N) P.c[m * P.c_ld + col] = acc[e];
    }
}

// ---------------------------------------------------------------- SF

struct SfParams {
    const float *s;
    uint16_t *p;
    float *m;
    float *l;
    int64_t s_ld, p_ld, m_st, l_st;
    int32_t M, valid, N;
    float scale;
};

__global__ void __launch_bounds__(256) tg_softmax_prepare_kernel(const SfParams P) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (row >= P.M) return;
    const float *s = P.s + row * P.s_ld;
    uint16_t *p = P.p + row * P.p_ld;
    const int valid = P.valid < P.N ? P.valid : P.N;
    // the first SV scores of each lane stay in registers between the two passes
    // (N <= 64 * SV: one read of the row)
    constexpr int SV = 4;
    float xs[SV];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < SV; ++i) {
        const int c = lane + 64 * i;
        xs[i] = c < valid ? s[c] * P.scale : -INFINITY;
        mx = fmaxf(mx, xs[i]);
    }
    for (int c = lane + 64 * SV; c < P.N; c += 64) {
        const float x = c < valid ? s[c] * P.scale : -INFINITY;
        mx = fmaxf(mx, x);
    }
    mx = wave_max(mx);
    const bool any = valid > 0;
    const float m = any ? mx : kMaskedRowMax;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < SV; ++i) {
        const int c = lane + 64 * i;
        if (c < P.N) {
            const uint16_t pb = any ? f32_to_bf16_rne(expf(xs[i] - m)) : (uint16_t)0;
            p[c] = pb;
            sum += bf16_to_f32(pb);
        }
    }
    for (int c = lane + 64 * SV; c < P.N; c += 64) {
        const float x = c < valid ? s[c] * P.scale : -INFINITY;
        const uint16_t pb = any ? f32_to_bf16_rne(expf(x - m)) : (uint16_t)0;
        p[c] = pb;
        sum += bf16_to_f32(pb);
    }
    sum = wave_sum(sum);
    if (lane == 0) {
        P.m[row * P.m_st] = m;
        P.l[row * P.l_st] = sum;
    }
}

// ---------------------------------------------------------------- UP

struct UpParams {
    const float *mij, *lij, *oi_new;
    float *mi, *li, *oi;
    void *dst;
    int64_t mij_st, lij_st, mi_st, li_st, on_ld, oi_ld, dst_ld;
    int32_t M, D, dst_bf16, is_first, is_last;
};

__global__ void __launch_bounds__(256) tg_online_update_kernel(const UpParams P) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (row >= P.M) return;
    const float *on = P.oi_new + row * P.on_ld;
    float *oi = P.oi + row * P.oi_ld;
    const float mj = P.mij[row * P.mij_st], lj = P.lij[row * P.lij_st];
    float alpha = 0.f, beta = 1.f, m_new = mj, l_new = lj;
    if (!P.is_first) {
        const float m_old = P.mi[row * P.mi_st], l_old = P.li[row * P.li_st];
        m_new = fmaxf(m_old, mj);
        alpha = expf(m_old - m_new);
        beta = expf(mj - m_new);
        const float t = alpha * l_old;
        const float u = beta * lj;
        l_new = t + u;
    }
    for (int d = lane; d < P.D; d += 64) {
        float o;
        if (P.is_first) {
            o = on[d];
        } else {
            const float x = oi[d] * alpha;
            const float y = on[d] * beta;
            o = x + y;
        }
        if (P.is_first || !P.is_last) oi[d] = o;
        if (P.is_last) {
            const float v = o / l_new;
            if (P.dst_bf16)
                reinterpret_cast<uint16_t *>(P.dst)[row * P.dst_ld + d] = f32_to_bf16_rne(v);
            else
                reinterpret_cast<float *>(P.dst)[row * P.dst_ld + d] = v;
        }
    }
    if (lane == 0) {
        P.mi[row * P.mi_st] = m_new;
        P.li[row * P.li_st] = l_new;
    }
}

// ---------------------------------------------------------------- vector example

struct VecParams {
    const float *a, *b;
    float *c;
    int64_t n;
    float s;
    int32_t op;  // 0 add, 1 add scalar, 2 mul
};

__global__ void __launch_bounds__(256) tg_vector_kernel(const VecParams P) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < P.n; i += step) {
        const float x = P.a[i];
        P.c[i] = P.op == 0 ? x + P.b[i] : P.op == 1 ? x + P.s : x * P.b[i];
    }
}

// ---------------------------------------------------------------- zero fill

struct FillParams {
    char *base;
    int64_t ld_bytes;   // row stride in bytes
    int64_t row_bytes;  // bytes per row (a multiple of 2)
    int32_t rows;
};

__global__ void __launch_bounds__(256) tg_zero_fill_kernel(const FillParams P) {
    const int64_t halves = P.row_bytes / 2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (int64_t)P.rows * halves;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / halves, c = i - r * halves;
        reinterpret_cast<uint16_t *>(P.base + r * P.ld_bytes)[c] = 0;
    }
}

// ---------------------------------------------------------------- host side

int fail(char *why, size_t len, int code, const char *fmt, ...) __attribute__((format(printf, 4, 5)));
int fail(char *why, size_t len, int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    if (why && len) vsnprintf(why, len, fmt, ap);
    va_end(ap);
    return code;
}

uint64_t extent_elems(const SimplerChipTensor &t) {
    uint64_t last = 0;
    for (uint32_t d = 0; d < t.ndims; ++d) {
        if (t.shapes[d] == 0) return 0;
        last += (uint64_t)(t.shapes[d] - 1) * t.strides[d];
    }
    return last + 1;
}

uint64_t numel(const SimplerChipTensor &t) {
    uint64_t n = 1;
    for (uint32_t d = 0; d < t.ndims; ++d) n *= t.shapes[d];
    return n;
}

bool row_major(const SimplerChipTensor &t) {
    uint64_t expect = 1;
    for (int d = (int)t.ndims - 1; d >= 0; --d) {
        if (t.shapes[d] != 1 && t.strides[d] != expect) return false;
        expect *= t.shapes[d];
    }
    return true;
}

// A tensor viewed as a matrix [rows, cols] (1-D: [1, n]; 2-D as is; more
// dims: leading dims must be row-major-collapsible into rows).
struct Mat {
    char *base;
    int64_t rows, cols, ld;
};

bool as_matrix(const SimplerChipTensor &t, Mat &m) {
    const uint64_t esz = simpler_dtype_size(t.dtype);
    m.base = reinterpret_cast<char *>((uintptr_t)(t.buffer.addr + t.start_offset * esz));
    if (t.ndims == 0 || t.ndims > SIMPLER_MAX_TENSOR_DIMS) return false;
    if (t.strides[t.ndims - 1] != 1 && t.shapes[t.ndims - 1] != 1) return false;
    m.cols = t.shapes[t.ndims - 1];
    if (t.ndims == 1) {
        m.rows = 1;
        m.ld = m.cols;
        return true;
    }
    m.ld = t.strides[t.ndims - 2];
    m.rows = t.shapes[t.ndims - 2];
    // leading dims fold into rows when they continue the row stride
    for (int d = (int)t.ndims - 3; d >= 0; --d) {
        if (t.shapes[d] != 1 && (uint64_t)t.strides[d] != (uint64_t)t.strides[d + 1] * t.shapes[d + 1]) return false;
        m.rows *= t.shapes[d];
    }
    return true;
}

// A 1-D (or [M, 1]) vector of M elements with an element stride.
bool as_vector(const SimplerChipTensor &t, int64_t M, float **p, int64_t *st) {
    const uint64_t esz = simpler_dtype_size(t.dtype);
    *p = reinterpret_cast<float *>((uintptr_t)(t.buffer.addr + t.start_offset * esz));
    if (t.dtype != SIMPLER_DT_FLOAT32 || (int64_t)numel(t) != M) return false;
    *st = 1;
    for (uint32_t d = 0; d < t.ndims; ++d)
        if (t.shapes[d] != 1) *st = t.strides[d];
    return true;
}

bool in_bounds(const SimplerChipTensor &t) {
    if (t.buffer.size == 0) return true;  // size unknown: trust the caller
    const uint64_t esz = simpler_dtype_size(t.dtype);
    return (t.start_offset + extent_elems(t)) * esz <= t.buffer.size;
}

bool aligned16(const void *p, int64_t ld, uint64_t esz) {
    return ((uintptr_t)p % 16 == 0) && ((ld * (int64_t)esz) % 16 == 0);
}

template <typename P>
void set_launch(KernelLaunch *out, const void *func, unsigned grid, unsigned block, const P &params) {
    static_assert(sizeof(P) <= kMaxKernelParamBytes, "parameter block too large");
    out->func = func;
    out->grid = dim3(grid > 0 ? grid : 1, 1, 1);
    out->block = dim3(block, 1, 1);
    out->param_bytes = sizeof(P);
    memcpy(out->params, &params, sizeof(P));
}

}  // namespace

int incore_tensor_count(int32_t kernel) {
    switch (kernel) {
        case SIMPLER_HIP_K_QK_MATMUL: return 3;
        case SIMPLER_HIP_K_SOFTMAX_PREPARE: return 4;
        case SIMPLER_HIP_K_PV_MATMUL: return 3;
        case SIMPLER_HIP_K_ONLINE_UPDATE: return 7;
        case SIMPLER_HIP_K_VEC_ADD: return 3;
        case SIMPLER_HIP_K_VEC_ADD_SCALAR: return 2;
        case SIMPLER_HIP_K_VEC_MUL: return 3;
        case SIMPLER_HIP_K_ZERO_FILL: return 1;
        default: return -1;
    }
}

int make_incore_launch(int32_t kernel, const SimplerChipTensor *t, int32_t nt, const uint64_t *s, int32_t ns,
                       KernelLaunch *out, char *why, size_t wl) {
    const int want = incore_tensor_count(kernel);
    if (want < 0) return fail(why, wl, SIMPLER_HIP_ERR_UNSUPPORTED, "unknown incore kernel %d", kernel);
    if (nt < want) return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "kernel %d needs %d tensors, got %d", kernel, want, nt);
    for (int i = 0; i < want; ++i) {
        if (t[i].ndims == 0 || t[i].ndims > SIMPLER_MAX_TENSOR_DIMS || simpler_dtype_size(t[i].dtype) == 0)
            return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "tensor %d: bad ndims/dtype", i);
        if (!in_bounds(t[i])) return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "tensor %d: view exceeds its buffer", i);
    }
    switch (kernel) {
        case SIMPLER_HIP_K_QK_MATMUL:
        case SIMPLER_HIP_K_PV_MATMUL: {
            const bool qk = kernel == SIMPLER_HIP_K_QK_MATMUL;
            Mat a, b, c;
            if (t[0].dtype != SIMPLER_DT_BFLOAT16 || t[1].dtype != SIMPLER_DT_BFLOAT16 ||
                t[2].dtype != SIMPLER_DT_FLOAT32)
                return fail(why, wl, SIMPLER_HIP_ERR_UNSUPPORTED, "%s: operands bf16, result fp32",
                            qk ? "qk_matmul" : "pv_matmul");
            if (!as_matrix(t[0], a) || !as_matrix(t[1], b) || !as_matrix(t[2], c))
                return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "matmul operands must be matrices with unit column stride");
            // QK: a [M,K], b [N,K]; PV: a [M,K], b [K,N]
            const int64_t M = a.rows, K = a.cols, N = qk ? b.rows : b.cols;
            if ((qk ? b.cols : b.rows) != K || c.rows != M || c.cols != N)
                return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "matmul shapes disagree (M=%lld K=%lld N=%lld)",
                            (long long)M, (long long)K, (long long)N);
            if (K % 8 != 0 || !aligned16(a.base, a.ld, 2) || (qk && !aligned16(b.base, b.ld, 2)))
                return fail(why, wl, SIMPLER_HIP_ERR_UNSUPPORTED,
                            "matmul needs K %% 8 == 0 and 16-byte aligned bf16 rows");
            MatParams P{reinterpret_cast<const uint16_t *>(a.base), reinterpret_cast<const uint16_t *>(b.base),
                        reinterpret_cast<float *>(c.base), a.ld, b.ld, c.ld, (int32_t)M, (int32_t)N, (int32_t)K};
            const int64_t tiles = ((M + 15) / 16) * ((N + 15) / 16);
            set_launch(out,
                       qk ? reinterpret_cast<const void *>(tg_matmul_kernel<true>)
                          : reinterpret_cast<const void *>(tg_matmul_kernel<false>),
                       (unsigned)((tiles + 3) / 4), 256, P);
            return SIMPLER_HIP_OK;
        }
        case SIMPLER_HIP_K_SOFTMAX_PREPARE: {
            Mat sv, p;
            if (t[0].dtype != SIMPLER_DT_FLOAT32 || t[1].dtype != SIMPLER_DT_BFLOAT16)
                return fail(why, wl, SIMPLER_HIP_ERR_UNSUPPORTED, "softmax_prepare: sij fp32, pij bf16");
            if (!as_matrix(t[0], sv) || !as_matrix(t[1], p))
                return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "softmax_prepare: sij/pij must be matrices");
            const int64_t M = p.rows, N = p.cols;
            if (sv.rows != M || sv.cols > N)
                return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "softmax_prepare: sij view [%lld,%lld] vs pij [%lld,%lld]",
                            (long long)sv.rows, (long long)sv.cols, (long long)M, (long long)N);
            float *m = nullptr, *l = nullptr;
            int64_t mst = 1, lst = 1;
            if (!as_vector(t[2], M, &m, &mst) || !as_vector(t[3], M, &l, &lst))
                return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "softmax_prepare: mij/lij must be fp32 [M]");
            if (ns < 1) return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "softmax_prepare: scale scalar missing");
            float scale;
            const uint32_t bits = (uint32_t)(s[0] & 0xffffffffu);
            memcpy(&scale, &bits, 4);
            // the valid columns are the view's width; the reference reads the
            // full [M, N] tile behind it (aiv_softmax_prepare.cpp:49,89-98)
            SfParams P{reinterpret_cast<const float *>(sv.base), reinterpret_cast<uint16_t *>(p.base), m, l,
                       sv.ld, p.ld, mst, lst, (int32_t)M, (int32_t)sv.cols, (int32_t)N, scale};
            set_launch(out, reinterpret_cast<const void *>(tg_softmax_prepare_kernel), (unsigned)((M + 3) / 4), 256, P);
            return SIMPLER_HIP_OK;
        }
        case SIMPLER_HIP_K_ONLINE_UPDATE: {
            Mat on, oi, dst;
            if (!as_matrix(t[2], on) || !as_matrix(t[5], oi) || !as_matrix(t[6], dst) ||
                t[2].dtype != SIMPLER_DT_FLOAT32 || t[5].dtype != SIMPLER_DT_FLOAT32 ||
                (t[6].dtype != SIMPLER_DT_FLOAT32 && t[6].dtype != SIMPLER_DT_BFLOAT16))
                return fail(why, wl, SIMPLER_HIP_ERR_INVALID,
                            "online_update: oi_new/oi fp32 matrices, dst fp32 or bf16 matrix");
            const int64_t M = on.rows, D = on.cols;
            if (oi.rows != M || oi.cols != D || dst.rows != M || dst.cols != D)
                return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "online_update: oi_new/oi/dst shapes disagree");
            UpParams P{};
            float *v[4];
            int64_t st[4];
            for (int i = 0; i < 4; ++i) {
                const int ti = i < 2 ? i : i + 1;  // mij, lij, mi, li
                if (!as_vector(t[ti], M, &v[i], &st[i]))
                    return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "online_update: tensor %d must be fp32 [M]", ti);
            }
            if (ns < 2) return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "online_update: is_first/is_last scalars missing");
            P.mij = v[0];
            P.lij = v[1];
            P.mi = v[2];
            P.li = v[3];
            P.mij_st = st[0];
            P.lij_st = st[1];
            P.mi_st = st[2];
            P.li_st = st[3];
            P.oi_new = reinterpret_cast<const float *>(on.base);
            P.oi = reinterpret_cast<float *>(oi.base);
            P.dst = dst.base;
            P.on_ld = on.ld;
            P.oi_ld = oi.ld;
            P.dst_ld = dst.ld;
            P.M = (int32_t)M;
            P.D = (int32_t)D;
            P.dst_bf16 = t[6].dtype == SIMPLER_DT_BFLOAT16;
            P.is_first = s[0] != 0;
            P.is_last = s[1] != 0;
            set_launch(out, reinterpret_cast<const void *>(tg_online_update_kernel), (unsigned)((M + 3) / 4), 256, P);
            return SIMPLER_HIP_OK;
        }
        case SIMPLER_HIP_K_VEC_ADD:
        case SIMPLER_HIP_K_VEC_ADD_SCALAR:
        case SIMPLER_HIP_K_VEC_MUL: {
            const int op = kernel == SIMPLER_HIP_K_VEC_ADD ? 0 : kernel == SIMPLER_HIP_K_VEC_ADD_SCALAR ? 1 : 2;
            const SimplerChipTensor &c = t[want - 1];
            const uint64_t n = numel(t[0]);
            for (int i = 0; i < want; ++i)
                if (t[i].dtype != SIMPLER_DT_FLOAT32 || !row_major(t[i]) || numel(t[i]) != n)
                    return fail(why, wl, SIMPLER_HIP_ERR_INVALID,
                                "vector kernels take contiguous fp32 tensors of equal size");
            if (op == 1 && ns < 1) return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "add_scalar: scalar missing");
            VecParams P{};
            P.a = reinterpret_cast<const float *>((uintptr_t)(t[0].buffer.addr + t[0].start_offset * 4));
            P.b = op == 1 ? nullptr
                          : reinterpret_cast<const float *>((uintptr_t)(t[1].buffer.addr + t[1].start_offset * 4));
            P.c = reinterpret_cast<float *>((uintptr_t)(c.buffer.addr + c.start_offset * 4));
            P.n = (int64_t)n;
            if (op == 1) {
                const uint32_t bits = (uint32_t)(s[0] & 0xffffffffu);
                memcpy(&P.s, &bits, 4);
            }
            P.op = op;
            const uint64_t blocks = (n + 255) / 256;
            set_launch(out, reinterpret_cast<const void *>(tg_vector_kernel), (unsigned)(blocks < 2048 ? blocks : 2048),
                       256, P);
            return SIMPLER_HIP_OK;
        }
        case SIMPLER_HIP_K_ZERO_FILL: {
            Mat d;
            if ((t[0].dtype != SIMPLER_DT_FLOAT32 && t[0].dtype != SIMPLER_DT_BFLOAT16) || !as_matrix(t[0], d))
                return fail(why, wl, SIMPLER_HIP_ERR_INVALID, "zero_fill: dst must be an fp32 or bf16 matrix");
            const int64_t esz = (int64_t)simpler_dtype_size(t[0].dtype);
            FillParams P{d.base, d.ld * esz, d.cols * esz, (int32_t)d.rows};
            const int64_t n = d.rows * d.cols * esz / 2;
            const int64_t blocks = (n + 255) / 256;
            set_launch(out, reinterpret_cast<const void *>(tg_zero_fill_kernel),
                       (unsigned)(blocks < 1024 ? blocks : 1024), 256, P);
            return SIMPLER_HIP_OK;
        }
        default: break;
    }
    return fail(why, wl, SIMPLER_HIP_ERR_UNSUPPORTED, "unknown incore kernel %d", kernel);
}

}  // namespace simpler_hip
