// Host side of the paged-attention decode: argument validation, the work
// plan (worker count, work lists, workspace layout), kernel selection and the
// C entry points of include/simpler_hip/pa_decode.h. The kernels themselves
// are in pa_kernels.h, instantiated by the pa_kernels_*.hip translation units.

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "simpler_hip/pa_decode.h"
#include "pa_decode_internal.h"
#include "pa_kernels.h"

namespace simpler_hip {
namespace {

using namespace pa;

// ----------------------------------------------------------------------------
// Host side: validation, worker count, dispatch
// ----------------------------------------------------------------------------

constexpr int kZeroOffset = 128;  // workspace bytes [128, 256) are never written after init
constexpr int kMaxAppendTokens = 16;  // fused append: new tokens per sequence (one per residue mod 16)
constexpr size_t kMaxZeroPageBytes = 1 << 20;  // larger token strides read the padding tiles as they are
constexpr int kMlaSegTokens = 256;  // MLA: work charged for each sequence a slice starts, in tokens

struct Plan {
    int workers;
    int row_tiles;
    int rows;
    int tiles_per_worker;
    int row_groups;
    int threads;  // per worker workgroup
    size_t lds;   // dynamic LDS per workgroup (sibling waves' K buffers)
    int groups;   // workgroups per worker (MLA row groups), else 1
    int lanes;    // work lists (KernelParams::lanes)
    int seg_cost; // KernelParams::seg_cost
    int64_t grid;
    KernelFn main;
    size_t flag_bytes, zero_bytes, part_ml_bytes, part_o_bytes;
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
    if (a->kv_format != SIMPLER_HIP_KV_BF16 && a->kv_format != SIMPLER_HIP_KV_FP8_E4M3 &&
        a->kv_format != SIMPLER_HIP_KV_FP16)
        return SIMPLER_HIP_ERR_INVALID;
    const bool fp8 = a->kv_format == SIMPLER_HIP_KV_FP8_E4M3;
    const int esz = fp8 ? 1 : 2;
    for (int64_t s : strides)
        if (s <= 0 || (s * esz) % 16) return SIMPLER_HIP_ERR_INVALID;  // 16-byte aligned rows
    if (a->k_token_stride * esz * a->block_size >= (int64_t)1 << 31 ||
        a->v_token_stride * esz * a->block_size >= (int64_t)1 << 31)
        return SIMPLER_HIP_ERR_INVALID;  // per-lane 32-bit byte offsets within a block
    if (fp8 && (!a->k_scale || !a->v_scale || ((uintptr_t)a->k_scale & 3) || ((uintptr_t)a->v_scale & 3)))
        return SIMPLER_HIP_ERR_INVALID;
    if (a->out_dtype != SIMPLER_HIP_DT_FLOAT32 && a->out_dtype != SIMPLER_HIP_DT_BFLOAT16 &&
        a->out_dtype != SIMPLER_HIP_DT_FLOAT16)
        return SIMPLER_HIP_ERR_UNSUPPORTED;
    if (!(a->scale == a->scale)) return SIMPLER_HIP_ERR_INVALID;
    if (a->num_workers < 0) return SIMPLER_HIP_ERR_INVALID;
    if (((uintptr_t)a->query | (uintptr_t)a->key_cache | (uintptr_t)a->value_cache | (uintptr_t)a->out) & 15)
        return SIMPLER_HIP_ERR_INVALID;
    const int group = a->num_heads / a->num_kv_heads;
    const int64_t row_tiles = ((int64_t)group * a->q_len + 15) / 16;
    // the flattened (tile, block) work list is indexed with 32-bit integers
    if ((int64_t)a->batch * a->num_kv_heads * row_tiles * a->max_blocks_per_seq >= (int64_t)1 << 31)
        return SIMPLER_HIP_ERR_UNSUPPORTED;
    if ((int64_t)a->batch * a->num_kv_heads * row_tiles >= (int64_t)1 << 31) return SIMPLER_HIP_ERR_UNSUPPORTED;
    return SIMPLER_HIP_OK;
}

// MLA: V is the first head_dim_v dims of K (same buffer, same strides).
bool is_mla_shape(const SimplerHipPaDecodeArgs *a) { return a->head_dim_k == kMlaDk && a->head_dim_v == kMlaDv; }

bool v_is_k_prefix(const SimplerHipPaDecodeArgs *a) {
    return a->value_cache == a->key_cache && a->v_block_stride == a->k_block_stride &&
           a->v_token_stride == a->k_token_stride && a->v_head_stride == a->k_head_stride;
}

// The main kernel(s) and the merge kernel a decode with these args runs;
// main is null when the combination is not supported. With `append`, ka holds
// the fused-append variants of k (same launch shapes; the plan is made from k).
struct Kernels {
    KernelPair k;
    KernelPair ka;
    MergeFn merge;
};

Kernels pick_kernel(const SimplerHipPaDecodeArgs *a, bool append = false) {
    Kernels s{};
    const int bs = a->block_size, dk = a->head_dim_k, dv = a->head_dim_v, out = a->out_dtype;
    const bool f16 = a->kv_format == SIMPLER_HIP_KV_FP16;
    if (a->kv_format == SIMPLER_HIP_KV_FP8_E4M3) {
        if (dk == dv && !append) s.k = pick_gqa_fp8(bs, dk, out);  // no fused append for fp8 caches
    } else if (is_mla_shape(a)) {
        // (the kernel's fill offsets use 24-bit multiplies: token rows below 8 MB)
        if (v_is_k_prefix(a) && a->kv_format == SIMPLER_HIP_KV_BF16 && a->k_token_stride * 2 < (1 << 23)) {
            s.k = pick_mla(bs, out);  // no fused form: the append runs as its own launch
        }
    } else if (dk == dv) {
        s.k = f16 ? pick_gqa_f16(bs, dk, out) : pick_gqa_bf16(bs, dk, out);
        if (append) s.ka = f16 ? pick_gqa_f16_append(bs, dk, out) : pick_gqa_bf16_append(bs, dk, out);
    }
    s.merge = pick_merge(dv, out);
    if (!s.merge.fn || (append && !s.ka.main)) s.k.main = nullptr;
    return s;
}

// Default worker count: compute units x the requested workgroups per CU,
// capped by what the kernel's register footprint allows. Kernels that read K
// in half lines (plain loads that rely on the L1 to merge the two halves)
// measured fastest at two waves per CU (512 workers: 112.8 us on the Qwen3-8B
// bs=32 shape, against 119.2 us with four per CU, whose K streams evict each
// other's L1 lines). Kernels that read K in whole rows and fp8 caches ask for
// four (one per SIMD).
// Without a device (host-only builds and tests) an MI355X is assumed:
// 256 CUs.
int wave_slots(KernelFn fn, int threads, int want_per_cu, size_t lds = 0) {
    struct Entry {
        KernelFn fn;
        int device;
        int threads;
        int want;
        size_t lds;
        int slots;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    std::lock_guard<std::mutex> lk(mu);
    for (const Entry &e : cache)
        if (e.fn == fn && e.device == dev && e.threads == threads && e.want == want_per_cu && e.lds == lds)
            return e.slots;
    // kWorkersPerCu workgroups per CU, or as many as fit (a 4-wave workgroup
    // fills a CU at one wave per SIMD). Two 2-wave workers per CU measured
    // 195.5 us on the speculative-verify shape against 213.9 us with one.
    int per_cu = want_per_cu;
    int cus = 256;
    // Without a device: the kernels use the whole register file of a SIMD
    // (one wave per SIMD, four SIMDs per CU), the MLA kernel most of the LDS.
    const int fit = 256 / threads;
    if (fit < per_cu) per_cu = fit > 0 ? fit : 1;
    if (dev >= 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(fn),
                                                         threads, lds) == hipSuccess &&
            n > 0 && n < per_cu)
            per_cu = n;
    }
    (void)hipGetLastError();
    const int slots = cus * per_cu;
    cache.push_back({fn, dev, threads, want_per_cu, lds, slots});
    return slots;
}

Plan make_plan(const SimplerHipPaDecodeArgs *a, const KernelPair &k) {  // k: the main kernels of pick_kernel
    Plan p{};
    const int group = a->num_heads / a->num_kv_heads;
    p.rows = group * a->q_len;
    p.row_tiles = (p.rows + 15) / 16;
    p.lanes = 1;
    if (k.mla) {
        // A work slice runs as `groups` sibling workgroups of 128 rows (8 row
        // tiles of 16) each; `workers` counts slices.
        p.groups = (p.rows + kMlaRowsPerGroup - 1) / kMlaRowsPerGroup;
        p.tiles_per_worker = kMlaRowsPerGroup / 16 * p.groups;
        p.row_groups = 1;
        p.threads = 256;
        p.main = k.main;
        if (a->num_workers > 0) {
            p.workers = a->num_workers;
        } else {
            const int wgs = wave_slots(p.main, p.threads, kWorkersPerCu);
            p.workers = wgs / p.groups > 0 ? wgs / p.groups : 1;
        }
        p.grid = (int64_t)p.workers * p.groups;
        // A slice that starts another sequence pays for its set-up: 147 KB of
        // query rows, a first block fetched without prefetch and a 256 KB
        // partial or output store, about 23 us per extra sequence on cfg4
        // (per-workgroup timestamps: 228 / 252 / 275 us for slices of one,
        // two and three sequences with equal blocks), so each sequence is
        // charged kMlaSegTokens tokens of work ahead of its blocks.
        p.seg_cost = (kMlaSegTokens + a->block_size - 1) / a->block_size;
    } else {
        // Row tiles of one kv head run as sibling waves of one worker workgroup
        // (up to four), so K/V of a block is fetched once for all of them;
        // two row tiles with K through LDS run in one wave instead.
        const bool pair = k.main_pair && p.row_tiles == 2;
        p.tiles_per_worker = pair ? 2 : (p.row_tiles < kMaxWavesPerWorker ? p.row_tiles : kMaxWavesPerWorker);
        p.threads = pair ? 64 : 64 * p.tiles_per_worker;
        p.main = pair ? k.main_pair : p.tiles_per_worker > 1 ? k.main_multi : k.main;
        if (!pair && k.klds && p.tiles_per_worker > 1) p.lds = (size_t)p.tiles_per_worker * a->block_size * 256;
        p.groups = 1;
        p.row_groups = (p.row_tiles + p.tiles_per_worker - 1) / p.tiles_per_worker;
        // One worker per SIMD when K is read in whole rows (through LDS); three
        // per CU for fp8 caches and for two-tile waves, whose blocks take
        // twice the math per byte (same-box medians at 768 against 1024
        // workers: fp8 57.4 against 58.7 us, the verify shape 134.2 against
        // 142.9; the single-tile kernel 108.2 against 108.9 on cfg2 but 165.5
        // against 164.5 on cfg3, so it keeps four); two per CU when K is read
        // in half lines, whose plain loads rely on the L1 merging the two
        // halves and evict each other at four.
        const bool fp8_kv = a->kv_format == SIMPLER_HIP_KV_FP8_E4M3;
        const int per_cu = (fp8_kv || pair) ? kWorkersThreePerCu
                           : (k.klds && p.main == k.main) ? kWorkersPerSimdCu
                                                          : kWorkersPerCu;
        p.workers = a->num_workers > 0 ? a->num_workers : wave_slots(p.main, p.threads, per_cu, p.lds);
        // Work lists (the tiles of a batch shared out among them, rotating with
        // the batch). 16-bit caches: one list per tile of a batch when the
        // worker count allows it, so the kv heads' workers walk the same blocks
        // side by side (cfg3-like long contexts: 167.7 us against 173.4 us
        // with one list, and 176 with two tiles per list). fp8 caches, whose
        // heads are single 128-byte lines of a 1 KB token row: four lists
        // (60.5 us against 61.4 with one list and 62.4 with one per tile on
        // the Qwen3-8B bs=32 shape).
        const int tpb = a->num_kv_heads * p.row_groups;
        const bool fp8 = a->kv_format == SIMPLER_HIP_KV_FP8_E4M3;
        const int want_lanes = fp8 ? (tpb % 4 == 0 ? 4 : 1) : tpb;
        if (want_lanes > 1) {
            if (a->num_workers > 0) {
                if (p.workers % want_lanes == 0) p.lanes = want_lanes;
            } else if (p.workers >= 4 * want_lanes) {
                p.workers -= p.workers % want_lanes;
                p.lanes = want_lanes;
            }
        }
        p.grid = p.workers;
    }
    const int dv = a->head_dim_v;
    // Layout: [error word] [zero page] [m,l partials] [O partials]; two
    // partial slots per worker wave. The zero page covers the lane offsets of
    // one 16-token tile (16 token strides of K or V, plus the dims): tiles past
    // a context's end read it instead of the cache. Its contents do not affect
    // results (those tokens are masked and their V rows zeroed), so calls of
    // other shapes may overwrite it.
    const int esz = a->kv_format == SIMPLER_HIP_KV_FP8_E4M3 ? 1 : 2;
    const size_t tok_bytes = (size_t)std::max(a->k_token_stride, a->v_token_stride) * esz;
    const size_t zero_bytes = align_up(16 * tok_bytes + 512, 256);
    p.zero_bytes = (!k.mla && zero_bytes <= kMaxZeroPageBytes) ? zero_bytes : 0;
    const size_t pieces = (size_t)p.workers * p.tiles_per_worker * 2;
    p.flag_bytes = 256;  // error word at 0, zeros at [kZeroOffset, 256)
    p.part_ml_bytes = align_up(pieces * 32 * sizeof(float), 256);
    p.part_o_bytes = align_up(pieces * 16 * dv * sizeof(float), 256);
    p.total = p.flag_bytes + p.zero_bytes + p.part_ml_bytes + p.part_o_bytes;
    return p;
}

}  // namespace
}  // namespace simpler_hip

using namespace simpler_hip;

extern "C" size_t simpler_hip_pa_decode_workspace_size(const SimplerHipPaDecodeArgs *args) {
    if (validate(args) != SIMPLER_HIP_OK) return 0;
    const Kernels s = pick_kernel(args);
    if (!s.k.main) return 0;
    return make_plan(args, s.k).total;
}

namespace simpler_hip {
namespace {
// Zeroes [p, p + bytes): 16-byte stores over the aligned body, byte stores for
// the tail. A kernel rather than hipMemsetAsync, so that callers may enqueue it
// inside a HIP graph capture (memset nodes are avoided in captured work).
__global__ void __launch_bounds__(256) zero_fill_kernel(char *p, size_t bytes) {
    const size_t n16 = bytes / 16;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        reinterpret_cast<u32x4_t *>(p)[i] = (u32x4_t){0u, 0u, 0u, 0u};
    if (blockIdx.x == 0 && threadIdx.x < bytes % 16) p[n16 * 16 + threadIdx.x] = 0;
}
}  // namespace

int zero_fill(void *p, size_t bytes, void *stream) {
    if (bytes == 0) return SIMPLER_HIP_OK;
    const size_t units = (bytes + 15) / 16;
    const unsigned grid = (unsigned)std::min<size_t>((units + 255) / 256, 2048);
    hipLaunchKernelGGL(zero_fill_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (char *)p, bytes);
    return hipGetLastError() == hipSuccess ? SIMPLER_HIP_OK : SIMPLER_HIP_ERR_LAUNCH;
}
}  // namespace simpler_hip

extern "C" int simpler_hip_pa_decode_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
    if (!workspace) return SIMPLER_HIP_ERR_WORKSPACE;
    return simpler_hip::zero_fill(workspace, workspace_bytes, stream);
}

extern "C" int simpler_hip_pa_decode_plan(const SimplerHipPaDecodeArgs *args, int32_t *num_workers) {
    const int rc = validate(args);
    if (rc != SIMPLER_HIP_OK) return rc;
    const Kernels s = pick_kernel(args);
    if (!s.k.main) return SIMPLER_HIP_ERR_UNSUPPORTED;
    if (num_workers) *num_workers = make_plan(args, s.k).workers;
    return SIMPLER_HIP_OK;
}

extern "C" const char *simpler_hip_pa_decode_kernel_name(const SimplerHipPaDecodeArgs *args) {
    if (validate(args) != SIMPLER_HIP_OK) return "";
    const Kernels s = pick_kernel(args);
    if (!s.k.main) return "";
    return s.k.mla ? "pa_mla_kernel" : "pa_decode_kernel";
}

extern "C" int simpler_hip_pa_decode(const SimplerHipPaDecodeArgs *a, void *workspace, size_t workspace_bytes,
                                     void *stream) {
    return simpler_hip_pa_decode_phase(a, workspace, workspace_bytes, stream,
                                       SIMPLER_HIP_PHASE_MAIN | SIMPLER_HIP_PHASE_MERGE);
}

namespace simpler_hip {
namespace {
// k_new / v_new: the fused append's new tokens (null: plain decode).
int pa_decode_launch(const SimplerHipPaDecodeArgs *a, void *workspace, size_t workspace_bytes, void *stream,
                     int phases, unsigned *err_mirror, const void *k_new = nullptr, const void *v_new = nullptr) {
    if (phases & ~(SIMPLER_HIP_PHASE_MAIN | SIMPLER_HIP_PHASE_MERGE)) return SIMPLER_HIP_ERR_INVALID;
    int rc = validate(a);
    if (rc != SIMPLER_HIP_OK) return rc;
    const bool append = k_new != nullptr;
    const Kernels s = pick_kernel(a, append);
    if (!s.k.main) return SIMPLER_HIP_ERR_UNSUPPORTED;
    Plan plan = make_plan(a, s.k);
    if (append)
        plan.main = plan.main == s.k.main_multi ? s.ka.main_multi : plan.main == s.k.main_pair ? s.ka.main_pair : s.ka.main;
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
    P.zeros = ws + kZeroOffset;
    P.zero_page = plan.zero_bytes ? ws + plan.flag_bytes : nullptr;
    P.part_ml = (float *)(ws + plan.flag_bytes + plan.zero_bytes);
    P.part_o = (float *)(ws + plan.flag_bytes + plan.zero_bytes + plan.part_ml_bytes);
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
    P.tiles_per_worker = plan.tiles_per_worker;
    P.row_groups = plan.row_groups;
    P.block_size = a->block_size;
    P.max_blocks = a->max_blocks_per_seq;
    P.num_pool_blocks = a->num_blocks;
    P.workers = plan.workers;
    P.lanes = plan.lanes;
    P.seg_cost = plan.seg_cost;
    P.scale = a->scale;
    P.causal = (a->causal && a->q_len > 1) ? 1 : 0;
    P.k_scale = a->k_scale;
    P.v_scale = a->v_scale;
    P.err_mirror = (phases & SIMPLER_HIP_PHASE_MERGE) ? err_mirror : nullptr;
    P.k_new = (const uint16_t *)k_new;
    P.v_new = (const uint16_t *)v_new;

    const int64_t tiles = (int64_t)a->batch * a->num_kv_heads * plan.row_tiles;
    if (phases & SIMPLER_HIP_PHASE_MAIN) {
        hipLaunchKernelGGL(plan.main, dim3((unsigned)plan.grid), dim3((unsigned)plan.threads), (unsigned)plan.lds,
                           (hipStream_t)stream, P);
        if (hipGetLastError() != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    }
    if (phases & SIMPLER_HIP_PHASE_MERGE) {
        hipLaunchKernelGGL(s.merge.fn, dim3((unsigned)tiles), dim3((unsigned)s.merge.threads), 0, (hipStream_t)stream,
                           P);
        if (hipGetLastError() != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    }
    return SIMPLER_HIP_OK;
}
}  // namespace

int pa_decode_with_mirror(const SimplerHipPaDecodeArgs *a, void *workspace, size_t workspace_bytes, void *stream,
                          unsigned *err_mirror) {
    return pa_decode_launch(a, workspace, workspace_bytes, stream, SIMPLER_HIP_PHASE_MAIN | SIMPLER_HIP_PHASE_MERGE,
                            err_mirror);
}
}  // namespace simpler_hip

extern "C" int simpler_hip_pa_decode_phase(const SimplerHipPaDecodeArgs *a, void *workspace, size_t workspace_bytes,
                                           void *stream, int phases) {
    return simpler_hip::pa_decode_launch(a, workspace, workspace_bytes, stream, phases, nullptr);
}

extern "C" int simpler_hip_pa_decode_append(const SimplerHipPaDecodeArgs *a, const void *key_new,
                                            const void *value_new, void *workspace, size_t workspace_bytes,
                                            void *stream) {
    const int rc = validate(a);
    if (rc != SIMPLER_HIP_OK) return rc;
    if (a->kv_format == SIMPLER_HIP_KV_FP8_E4M3 || a->q_len > kMaxAppendTokens) return SIMPLER_HIP_ERR_UNSUPPORTED;
    const bool mla = is_mla_shape(a) && v_is_k_prefix(a);
    if (!key_new || ((uintptr_t)key_new & 15)) return SIMPLER_HIP_ERR_INVALID;
    if (mla ? value_new != nullptr : (!value_new || ((uintptr_t)value_new & 15))) return SIMPLER_HIP_ERR_INVALID;
    {
        // Two or more row tiles per worker (the two-tile wave, sibling waves,
        // MLA's 128-row workgroups): the append runs as its own launch ahead
        // of the plain decode. There the fused form's unpipelined new-token
        // blocks measured slower (the verify shape: 155.2 against 140.2 us per
        // step), and MLA's register budget has no room for the new rows; with
        // one tile per worker the fused form is the faster one (cfg2: 113.3
        // against 114.5).
        const Kernels s = pick_kernel(a);
        if (s.k.main) {
            const Plan plan = make_plan(a, s.k);
            if (plan.tiles_per_worker > 1 || s.k.mla) {
                if (!workspace || workspace_bytes < plan.total || ((uintptr_t)workspace & 255))
                    return SIMPLER_HIP_ERR_WORKSPACE;
                if (a->batch == 0) return SIMPLER_HIP_OK;
                const int rc2 =
                    launch_paged_append(a, key_new, value_new, (unsigned *)workspace, kErrBadLength, stream);
                if (rc2 != SIMPLER_HIP_OK) return rc2;
                return pa_decode_launch(a, workspace, workspace_bytes, stream,
                                        SIMPLER_HIP_PHASE_MAIN | SIMPLER_HIP_PHASE_MERGE, nullptr);
            }
        }
    }
    return simpler_hip::pa_decode_launch(a, workspace, workspace_bytes, stream,
                                         SIMPLER_HIP_PHASE_MAIN | SIMPLER_HIP_PHASE_MERGE, nullptr, key_new,
                                         value_new);
}

namespace {

// simpler_hip_pa_decode_prelude's workspace after the decode's: the bf16
// query rows the prelude writes.
size_t prelude_query_bytes(const SimplerHipPaDecodeArgs *a) {
    return align_up((size_t)a->batch * a->q_len * a->num_heads * a->head_dim_k * 2, 256);
}

// The prelude entry's checks beyond validate(); a->query is not read.
int check_prelude(const SimplerHipPaDecodeArgs *a, const SimplerHipDecodePreludeArgs *pre) {
    if (a->kv_format != SIMPLER_HIP_KV_BF16 || a->head_dim_k != 128 || a->head_dim_v != 128 ||
        a->q_len > kMaxAppendTokens || (is_mla_shape(a) && v_is_k_prefix(a)))
        return SIMPLER_HIP_ERR_UNSUPPORTED;
    if (!pre) return SIMPLER_HIP_OK;
    const void *ptrs[8] = {pre->q_proj,        pre->k_proj,        pre->v_proj,   pre->inv_rms,
                           pre->q_norm_weight, pre->k_norm_weight, pre->rope_cos, pre->rope_sin};
    for (const void *p : ptrs)
        if (!p || ((uintptr_t)p & 15)) return SIMPLER_HIP_ERR_INVALID;
    if (pre->max_position < 1 || !(pre->eps >= 0.f)) return SIMPLER_HIP_ERR_INVALID;
    return SIMPLER_HIP_OK;
}

}  // namespace

extern "C" size_t simpler_hip_pa_decode_prelude_workspace_size(const SimplerHipPaDecodeArgs *a) {
    if (!a) return 0;
    SimplerHipPaDecodeArgs args = *a;
    if (!args.query) args.query = (const void *)(uintptr_t)256;  // not read: any aligned stand-in validates
    if (validate(&args) != SIMPLER_HIP_OK || check_prelude(&args, nullptr) != SIMPLER_HIP_OK) return 0;
    const Kernels s = pick_kernel(&args);
    if (!s.k.main) return 0;
    return make_plan(&args, s.k).total + prelude_query_bytes(&args);
}

extern "C" int simpler_hip_pa_decode_prelude(const SimplerHipPaDecodeArgs *a, const SimplerHipDecodePreludeArgs *pre,
                                             void *workspace, size_t workspace_bytes, void *stream) {
    if (!a || !pre) return SIMPLER_HIP_ERR_INVALID;
    // the query is computed: validate the rest with q_proj standing in for it
    SimplerHipPaDecodeArgs args = *a;
    args.query = pre->q_proj;
    int rc = validate(&args);
    if (rc != SIMPLER_HIP_OK) return rc;
    rc = check_prelude(&args, pre);
    if (rc != SIMPLER_HIP_OK) return rc;
    const Kernels s = pick_kernel(&args);
    if (!s.k.main) return SIMPLER_HIP_ERR_UNSUPPORTED;
    const size_t total = make_plan(&args, s.k).total;
    if (!workspace || workspace_bytes < total + prelude_query_bytes(&args) || ((uintptr_t)workspace & 255))
        return SIMPLER_HIP_ERR_WORKSPACE;
    if (args.batch == 0) return SIMPLER_HIP_OK;
    // The prelude as a launch of its own (query rows into the workspace after
    // the decode's part, new K/V rows into the caches), then the plain
    // decode on that query. Computing the prelude inside the decode's workers
    // measured slower on every shape tried (cfg2 117.4 against 115.6 us per
    // step, the verify shape 161.0 against 142.6, cfg1 17.5 against 14.3).
    void *const q = (char *)workspace + total;
    rc = launch_paged_prelude(&args, pre, q, (unsigned *)workspace, kErrBadLength, stream);
    if (rc != SIMPLER_HIP_OK) return rc;
    args.query = q;
    return simpler_hip::pa_decode_launch(&args, workspace, total, stream,
                                         SIMPLER_HIP_PHASE_MAIN | SIMPLER_HIP_PHASE_MERGE, nullptr);
}

// ---------------------------------------------------------------------------
// The entry point that allocates nothing: simpler_hip_pa_decode with the
// workspace replaced by a fixed device array of this library.
// ---------------------------------------------------------------------------

namespace simpler_hip {
namespace {

// Every decode of the direct entry fits here at the default worker count on
// MI355X (256 CUs): a GQA plan needs at most 2048 partial slots of 16 rows x
// Dv fp32 (Dv 128: 16 MiB, Dv 256: 32 MiB), the MLA plan 4096 slots of 16 x 512
// fp32 (256 slices x 8 row tiles x 2: 128 MiB), plus (m, l) pairs, the error
// word and the zero page.
constexpr size_t kScratchBytes = (size_t)SIMPLER_HIP_PA_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch size");

// One copy per GPU the library runs on, held until the process ends. In host
// code `scratch` is only a stand-in for the symbol: its device address comes
// from hipGetSymbolAddress, per device.
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxScratchDevices] = {};

// This device's address of `scratch`, looked up once per device (with that
// device current) and kept; nullptr if the lookup fails.
void *scratch_on_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace simpler_hip

extern "C" int simpler_hip_pa_decode_noalloc(const SimplerHipPaDecodeArgs *a, void *stream) {
    int rc = validate(a);
    if (rc != SIMPLER_HIP_OK) return rc;
    const Kernels s = pick_kernel(a);
    if (!s.k.main) return SIMPLER_HIP_ERR_UNSUPPORTED;
    const size_t need = make_plan(a, s.k).total;
    if (need > kScratchBytes) {
        fprintf(stderr,
                "[simpler_hip] simpler_hip_pa_decode_noalloc: this decode needs %zu bytes of scratch, above the "
                "fixed %zu (use fewer workers or simpler_hip_pa_decode with a workspace)\n",
                need, kScratchBytes);
        return SIMPLER_HIP_ERR_WORKSPACE;
    }
    void *ws = scratch_on_current_device();
    if (!ws) return SIMPLER_HIP_ERR_LAUNCH;
    // Nothing in the scratch has to start at zero: every partial slot the
    // merge reads is written by the same call's main kernel, and the zero
    // page's contents never reach a result. The error word only accumulates.
    return simpler_hip::pa_decode_launch(a, ws, kScratchBytes, stream, SIMPLER_HIP_PHASE_MAIN | SIMPLER_HIP_PHASE_MERGE,
                                         nullptr);
}

extern "C" int simpler_hip_pa_decode_check(void *workspace, size_t workspace_bytes, void *stream) {
    if (!workspace || workspace_bytes < sizeof(unsigned)) return SIMPLER_HIP_ERR_WORKSPACE;
    unsigned flag = 0;
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    if (hipMemcpy(&flag, workspace, sizeof(flag), hipMemcpyDeviceToHost) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    if (flag == 0) return SIMPLER_HIP_OK;
    const unsigned zero = 0;
    if (hipMemcpy(workspace, &zero, sizeof(zero), hipMemcpyHostToDevice) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    return (flag & kErrBadBlock) ? SIMPLER_HIP_ERR_BAD_BLOCK : SIMPLER_HIP_ERR_BAD_LENGTH;
}
