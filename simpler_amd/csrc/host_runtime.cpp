// libsimpler_hip.so host runtime: simpler's host-runtime C API on one HIP device.
//
// The reference's ChipWorker dlopens a host runtime and drives it through
// these symbols (src/common/worker/chip_worker.cpp:205-256). Here a device
// context owns one HIP stream, a device-memory ledger, a registry of up to 64
// callables and a grow-only workspace for the fused decode kernel.
//
// A paged-attention run reads its arguments the way the reference
// orchestration does (examples/a2a3/tensormap_and_ringbuffer/paged_attention/
// kernels/orchestration/paged_attention_orch.cpp:94-102): tensors
// 0..5 = query, key_cache, value_cache, block_table, context_lens, out and
// scalar 0 = softmax scale as fp32 bits. Optional scalar 1 = causal flag for a
// multi-token query (no reference counterpart).
//
// Host tensors are staged like the reference's stage_device_args
// (src/a2a3/runtime/tensormap_and_ringbuffer/host/runtime_maker.cpp:575-652):
// copied to the device unless the signature says OUT, copied back unless IN.
// Tensors whose address_space is DEVICE (tensor.h:105) pass through untouched.
//
// Execution of a paged-attention callable is the fused decode kernel by
// default. With the task-graph execution selected (simpler_hip_set_execution
// or SIMPLER_HIP_EXECUTION=eager|graph at init) the reference's orchestration
// runs instead, QK -> SF -> PV -> UP per KV block, on the task-graph backend
// (task_graph.h). The reference's vector example callable always runs there.

#include <hip/hip_runtime.h>

#include <memory>
#include <stdlib.h>
#include <mutex>
#include <new>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <unordered_map>
#include <vector>

#include "simpler_hip/abi_types.h"
#include "simpler_hip/pa_decode.h"
#include "simpler_hip/pto_runtime_c_api.h"
#include "simpler_hip/task_graph.h"
#include "pa_decode_internal.h"

namespace {

constexpr int kMaxCallables = 64;  // callable ids 0..63 (pto_runtime_c_api.h:285-287)
constexpr int kPaTensors = 6;
constexpr int kVecTensors = 3;
constexpr int kMaxRunTensors = 8;
constexpr uint32_t kRunMagic = 0x53485052u;  // "SHPR"
const char *const kNativePaName = "simpler_hip_paged_attention_decode";

void logf(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "[simpler_hip] ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
}

enum CallableKind { kNone = 0, kPagedAttention = 1, kVectorExample = 2 };

// Which of the reference's paged-attention callables a registration matched.
// All of them take the same orchestration arguments (query, key_cache,
// value_cache, block_table, context_lens, out; scalar 0 = scale) and compute
// the same golden, so the fused kernel serves every one; only kPaChain's
// orchestration is also available on the task-graph backend.
enum PaFamily {
    kPaChain = SIMPLER_HIP_PA_CHAIN,    // QK/SF/PV/UP per block: paged_attention, *_manual_scope, *_ringbuffer,
                                        // batch_*, multi_round_*
    kPaUnroll = SIMPLER_HIP_PA_UNROLL,  // grouped QK/SF/PV over <= 64 blocks + UP: paged_attention_unroll,
                                        // *_unroll_manual_scope, *_unroll_4dims
    kPaSpmd = SIMPLER_HIP_PA_SPMD,      // one cooperative AIC/AIV mix task: spmd_paged_attention
    kPaNative = SIMPLER_HIP_PA_NATIVE,  // the name simpler_hip_paged_attention_decode
    kPaHighperf = SIMPLER_HIP_PA_HIGHPERF,  // spmd_paged_attention_highperf: lengths and scale in a tiling tensor
};

struct Callable {
    CallableKind kind = kNone;
    int32_t family = kPaChain;
    int32_t sig[SIMPLER_CHIP_MAX_TENSOR_ARGS] = {};
    int32_t sig_count = 0;
};

struct DeviceContext {
    std::mutex mu;
    int device_id = -1;
    hipStream_t stream = nullptr;
    std::unordered_map<void *, size_t> allocs;
    size_t committed = 0;
    Callable callables[kMaxCallables];
    void *workspace = nullptr;
    size_t workspace_bytes = 0;
    size_t runs = 0;
    int32_t execution = SIMPLER_HIP_EXEC_FUSED;
    SimplerHipTaskGraph *graphs[2] = {nullptr, nullptr};  // eager, hipGraph
    // Completion event of the runs on `stream`, recorded anew by every launch.
    // Runs launched back to back share it, so waiting on an earlier one waits
    // for the later ones too: later, never too early.
    hipEvent_t done = nullptr;
    // Host copy of the decode workspace's error word in coherent pinned
    // memory, stored by each fused decode's merge kernel, so the wait reads it
    // from host memory instead of a stream synchronisation and a blocking copy.
    unsigned *err_host = nullptr;
};

// Native-run state lives in caller-owned storage of get_runtime_size() bytes
// (pto_runtime_c_api.h:43-49), zeroed before first use.
struct NativeRun {
    uint32_t magic;
    uint32_t state;  // 0 idle, 1 prepared, 2 launched
    int32_t callable_id;
    int32_t kind;       // CallableKind
    int32_t execution;  // SIMPLER_HIP_EXEC_* chosen at prepare
    int32_t n_tensors;
    int32_t n_staged;
    hipEvent_t done;  // the context's completion event (not owned by the run)
    void *staged_dev[kMaxRunTensors];
    void *host_ptr[kMaxRunTensors];
    size_t staged_bytes[kMaxRunTensors];
    int32_t dir[kMaxRunTensors];
    uint64_t scale_bits;
    int32_t *host_lens;  // highperf family: context lengths taken from the tiling tensor (malloc'd)
    SimplerChipTensor tensors[kMaxRunTensors];  // the run's tensors as device work sees them
    SimplerHipPaDecodeArgs args;
};

const PipelineContract kContract = {PTO_PIPELINE_CONTRACT_ABI_VERSION, 0, 1, {}};

DeviceContext *as_ctx(DeviceContextHandle h) { return static_cast<DeviceContext *>(h); }

bool set_device(DeviceContext *c) {
    if (!c || c->device_id < 0) return false;
    return hipSetDevice(c->device_id) == hipSuccess;
}

// --- callable recognition ----------------------------------------------------

// Signatures of the reference chain (test_paged_attention.py:25-61).
const int32_t kOrchSig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN,
                            SIMPLER_ARG_OUT};
const int32_t kQkSig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_OUT};
const int32_t kSfSig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_OUT, SIMPLER_ARG_OUT, SIMPLER_ARG_OUT};
const int32_t kPvSig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_OUT};
const int32_t kUpSig[] = {SIMPLER_ARG_IN,    SIMPLER_ARG_IN,    SIMPLER_ARG_IN,   SIMPLER_ARG_INOUT,
                          SIMPLER_ARG_INOUT, SIMPLER_ARG_INOUT, SIMPLER_ARG_INOUT};
// Grouped split-K chain (tests/st/a2a3/tensormap_and_ringbuffer/paged_attention_unroll/
// test_paged_attention_unroll.py:25-61, the same in paged_attention_unroll_4dims and
// examples/.../paged_attention_unroll_manual_scope): QK and PV take a third input.
const int32_t kQkUnrollSig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_OUT};
const int32_t kPvUnrollSig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_OUT};
// Cooperative AIC/AIV task (tests/st/a2a3/tensormap_and_ringbuffer/spmd_paged_attention/
// test_spmd_paged_attention.py:28-54): func ids 0 and 1 share one 9-tensor payload.
const int32_t kSpmdMixSig[] = {SIMPLER_ARG_IN,    SIMPLER_ARG_IN,  SIMPLER_ARG_IN,  SIMPLER_ARG_IN, SIMPLER_ARG_IN,
                               SIMPLER_ARG_INOUT, SIMPLER_ARG_OUT, SIMPLER_ARG_OUT, SIMPLER_ARG_OUT};

// The high-performance SPMD callable (tests/st/a2a3/tensormap_and_ringbuffer/
// spmd_paged_attention_highperf/test_spmd_paged_attention_highperf.py:96-165):
// query, key_cache, value_cache, block_table, out, eight workspaces, tiling,
// null; both halves of the mix task declare the same 15-tensor payload.
const int32_t kHighperfSig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_OUT,
                                SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN,
                                SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_IN};
constexpr int kHighperfTensors = 15;

struct ChildSig {
    const int32_t *sig;
    int32_t n;
};
struct PaFamilySpec {
    PaFamily family;
    int32_t children;       // func ids 0 .. children-1, each exactly once
    ChildSig by_fid[4];
};
const PaFamilySpec kPaFamilies[] = {
    {kPaChain, 4, {{kQkSig, 3}, {kSfSig, 4}, {kPvSig, 3}, {kUpSig, 7}}},
    {kPaUnroll, 4, {{kQkUnrollSig, 4}, {kSfSig, 4}, {kPvUnrollSig, 4}, {kUpSig, 7}}},
    {kPaSpmd, 2, {{kSpmdMixSig, 9}, {kSpmdMixSig, 9}, {nullptr, 0}, {nullptr, 0}}},
};
const PaFamilySpec kHighperfFamily = {
    kPaHighperf, 2, {{kHighperfSig, kHighperfTensors}, {kHighperfSig, kHighperfTensors}, {nullptr, 0}, {nullptr, 0}}};

bool sig_equals(const int32_t *a, int32_t na, const int32_t *b, int32_t nb) {
    if (na != nb) return false;
    for (int i = 0; i < na; ++i)
        if (a[i] != b[i]) return false;
    return true;
}

// The vector example (examples/a2a3/tensormap_and_ringbuffer/vector_example/
// test_vector_example.py:24-49): orchestration [IN, IN, OUT]; children
// 0 kernel_add [IN, IN, OUT], 1 kernel_add_scalar [IN, OUT], 2 kernel_mul [IN, IN, OUT].
const int32_t kVecOrchSig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_IN, SIMPLER_ARG_OUT};
const int32_t kVecUnarySig[] = {SIMPLER_ARG_IN, SIMPLER_ARG_OUT};

CallableKind classify_vector(const SimplerChipCallableHeader &h, const uint8_t *blob) {
    const uint8_t *storage = blob + SIMPLER_CHIP_CALLABLE_STORAGE_OFFSET;
    bool seen[3] = {false, false, false};
    for (int i = 0; i < 3; ++i) {
        const int fid = h.child_func_ids_[i];
        if (fid < 0 || fid > 2 || seen[fid]) return kNone;
        seen[fid] = true;
        SimplerCoreCallableHeader ch;
        memcpy(&ch, storage + h.child_offsets_[i], sizeof(ch));
        const bool ok = fid == 1 ? sig_equals(ch.signature_, ch.sig_count_, kVecUnarySig, 2)
                                 : sig_equals(ch.signature_, ch.sig_count_, kVecOrchSig, 3);
        if (!ok) return kNone;
    }
    return kVectorExample;
}

CallableKind classify(const uint8_t *blob, Callable &out) {
    SimplerChipCallableHeader h;
    memcpy(&h, blob, sizeof(h));
    if (h.sig_count_ < 0 || h.sig_count_ > SIMPLER_CHIP_MAX_TENSOR_ARGS) return kNone;
    if (h.child_count_ < 0 || h.child_count_ > SIMPLER_CHIP_MAX_CHILDREN) return kNone;
    out.sig_count = h.sig_count_;
    memcpy(out.sig, h.signature_, sizeof(int32_t) * h.sig_count_);
    char name[SIMPLER_CALLABLE_FUNC_NAME_MAX + 1] = {};
    memcpy(name, h.func_name_, SIMPLER_CALLABLE_FUNC_NAME_MAX);
    if (strcmp(name, kNativePaName) == 0 && h.sig_count_ >= kPaTensors) {
        out.family = kPaNative;
        return kPagedAttention;
    }
    if (sig_equals(h.signature_, h.sig_count_, kVecOrchSig, 3) && h.child_count_ == 3) return classify_vector(h, blob);
    const bool highperf = sig_equals(h.signature_, h.sig_count_, kHighperfSig, kHighperfTensors);
    if (!highperf && !sig_equals(h.signature_, h.sig_count_, kOrchSig, 6)) return kNone;
    // The paged-attention orchestrations: the children (in any order) must be
    // exactly one family's func ids with that family's signatures.
    const uint8_t *storage = blob + SIMPLER_CHIP_CALLABLE_STORAGE_OFFSET;
    const PaFamilySpec *families = highperf ? &kHighperfFamily : kPaFamilies;
    const int n_families = highperf ? 1 : (int)(sizeof(kPaFamilies) / sizeof(kPaFamilies[0]));
    for (int fi = 0; fi < n_families; ++fi) {
        const PaFamilySpec &f = families[fi];
        if (h.child_count_ != f.children) continue;
        bool seen[4] = {false, false, false, false};
        bool ok = true;
        for (int i = 0; i < f.children && ok; ++i) {
            const int fid = h.child_func_ids_[i];
            if (fid < 0 || fid >= f.children || seen[fid]) {
                ok = false;
                break;
            }
            seen[fid] = true;
            SimplerCoreCallableHeader ch;
            memcpy(&ch, storage + h.child_offsets_[i], sizeof(ch));
            ok = sig_equals(ch.signature_, ch.sig_count_, f.by_fid[fid].sig, f.by_fid[fid].n);
        }
        if (ok) {
            out.family = f.family;
            return kPagedAttention;
        }
    }
    return kNone;
}

// --- argument decoding -----------------------------------------------------------

const SimplerChipTensor &tensor_at(const SimplerChipStorageTaskArgs *a, int i) { return a->tensors_[i]; }

bool contiguous(const SimplerChipTensor &t) {
    uint64_t expect = 1;
    for (int d = (int)t.ndims - 1; d >= 0; --d) {
        if (t.shapes[d] != 1 && t.strides[d] != expect) return false;
        expect *= t.shapes[d];
    }
    return true;
}

uint64_t extent_bytes(const SimplerChipTensor &t) {
    uint64_t last = 0;
    for (uint32_t d = 0; d < t.ndims; ++d)
        if (t.shapes[d]) last += (uint64_t)(t.shapes[d] - 1) * t.strides[d];
    return (t.start_offset + last + 1) * simpler_dtype_size(t.dtype);
}

int decode_pa_args(const SimplerChipStorageTaskArgs *a, SimplerHipPaDecodeArgs &pa, int causal_scalar_index) {
    if (a->tensor_count_ < kPaTensors || a->scalar_count_ < 1) {
        logf("paged attention needs 6 tensors and a scale scalar (got %d tensors, %d scalars)", a->tensor_count_,
             a->scalar_count_);
        return SIMPLER_HIP_ERR_INVALID;
    }
    const SimplerChipTensor &q = tensor_at(a, 0), &k = tensor_at(a, 1), &v = tensor_at(a, 2);
    const SimplerChipTensor &bt = tensor_at(a, 3), &cl = tensor_at(a, 4), &o = tensor_at(a, 5);
    memset(&pa, 0, sizeof(pa));
    // fp8 caches: FP8E4M3FN key/value caches, then tensors 6 and 7 = fp32
    // [num_blocks, kv_heads] K and V scales (no reference counterpart)
    const bool fp8 = k.dtype == SIMPLER_DT_FP8E4M3FN;
    const bool fp16 = q.dtype == SIMPLER_DT_FLOAT16;
    const bool ok_dtypes = fp16 ? (k.dtype == SIMPLER_DT_FLOAT16 && v.dtype == SIMPLER_DT_FLOAT16)
                                : (q.dtype == SIMPLER_DT_BFLOAT16 && (fp8 || k.dtype == SIMPLER_DT_BFLOAT16) &&
                                   v.dtype == k.dtype);
    if (!ok_dtypes) {
        logf("query/key_cache/value_cache must be BFLOAT16 (caches BFLOAT16 or FP8E4M3FN) or all FLOAT16");
        return SIMPLER_HIP_ERR_UNSUPPORTED;
    }
    if (fp16) pa.kv_format = SIMPLER_HIP_KV_FP16;
    if (fp8) {
        if (a->tensor_count_ < kPaTensors + 2) {
            logf("fp8 caches need tensors 6 and 7: k_scale and v_scale, fp32 [num_blocks, kv_heads]");
            return SIMPLER_HIP_ERR_INVALID;
        }
        for (int i = kPaTensors; i < kPaTensors + 2; ++i) {
            const SimplerChipTensor &sc = tensor_at(a, i);
            if (sc.dtype != SIMPLER_DT_FLOAT32 || sc.ndims != 2 || !contiguous(sc) || sc.shapes[0] != k.shapes[0] ||
                sc.shapes[1] != (k.ndims == 4 ? k.shapes[2] : 1)) {
                logf("k_scale/v_scale must be contiguous fp32 [num_blocks, kv_heads]");
                return SIMPLER_HIP_ERR_INVALID;
            }
        }
        pa.kv_format = SIMPLER_HIP_KV_FP8_E4M3;
    }
    if (bt.dtype != SIMPLER_DT_INT32 || cl.dtype != SIMPLER_DT_INT32 || bt.ndims != 2 || cl.ndims != 1) {
        logf("block_table must be INT32 [B, max_blocks] and context_lens INT32 [B]");
        return SIMPLER_HIP_ERR_INVALID;
    }
    if (!contiguous(q) || !contiguous(bt) || !contiguous(cl) || !contiguous(o)) {
        logf("query, block_table, context_lens and out must be contiguous");
        return SIMPLER_HIP_ERR_INVALID;
    }
    int batch, q_len, hq, dk;
    if (q.ndims == 3) {
        batch = q.shapes[0]; q_len = 1; hq = q.shapes[1]; dk = q.shapes[2];
    } else if (q.ndims == 4) {
        batch = q.shapes[0]; q_len = q.shapes[1]; hq = q.shapes[2]; dk = q.shapes[3];
    } else {
        logf("query must be [B, Hq, D] or [B, q_len, Hq, D]");
        return SIMPLER_HIP_ERR_INVALID;
    }
    // key/value cache: [nblk, BS, Hkv, D] (BSND) or [nblk, BS, D] with one KV head
    auto kv_geom = [](const SimplerChipTensor &t, int &nblk, int &bs, int &hkv, int &d, int64_t (&st)[3]) {
        if (t.ndims == 4) {
            nblk = t.shapes[0]; bs = t.shapes[1]; hkv = t.shapes[2]; d = t.shapes[3];
            if (t.strides[3] != 1) return false;
            st[0] = t.strides[0]; st[1] = t.strides[1]; st[2] = t.strides[2];
        } else if (t.ndims == 3) {
            nblk = t.shapes[0]; bs = t.shapes[1]; hkv = 1; d = t.shapes[2];
            if (t.strides[2] != 1) return false;
            st[0] = t.strides[0]; st[1] = t.strides[1]; st[2] = d;
        } else {
            return false;
        }
        return true;
    };
    int knb, kbs, khkv, kd, vnb, vbs, vhkv, vd;
    int64_t kst[3], vst[3];
    if (!kv_geom(k, knb, kbs, khkv, kd, kst) || !kv_geom(v, vnb, vbs, vhkv, vd, vst)) {
        logf("key_cache/value_cache must be [num_blocks, block_size, kv_heads, head_dim] with unit dim stride");
        return SIMPLER_HIP_ERR_INVALID;
    }
    if (knb != vnb || kbs != vbs || khkv != vhkv || kd != dk) {
        logf("cache shapes disagree with each other or with the query head_dim");
        return SIMPLER_HIP_ERR_INVALID;
    }
    if ((int)bt.shapes[0] != batch || (int)cl.shapes[0] != batch) {
        logf("block_table/context_lens batch does not match the query");
        return SIMPLER_HIP_ERR_INVALID;
    }
    const bool out4 = o.ndims == 4;
    if (!((o.ndims == 3 && q_len == 1) || out4) || (int)o.shapes[0] != batch ||
        (int)o.shapes[o.ndims - 2] != hq || (int)o.shapes[o.ndims - 1] != vd || (out4 && (int)o.shapes[1] != q_len)) {
        logf("out must be [B, Hq, Dv] or [B, q_len, Hq, Dv]");
        return SIMPLER_HIP_ERR_INVALID;
    }
    pa.batch = batch;
    pa.q_len = q_len;
    pa.num_heads = hq;
    pa.num_kv_heads = khkv;
    pa.head_dim_k = dk;
    pa.head_dim_v = vd;
    pa.block_size = kbs;
    pa.max_blocks_per_seq = bt.shapes[1];
    pa.num_blocks = knb;
    pa.k_block_stride = kst[0]; pa.k_token_stride = kst[1]; pa.k_head_stride = kst[2];
    pa.v_block_stride = vst[0]; pa.v_token_stride = vst[1]; pa.v_head_stride = vst[2];
    pa.out_dtype = o.dtype;
    uint32_t bits = (uint32_t)(a->scalars_[0] & 0xffffffffu);
    memcpy(&pa.scale, &bits, 4);
    pa.causal = (causal_scalar_index < a->scalar_count_) ? (a->scalars_[causal_scalar_index] != 0) : 0;
    return SIMPLER_HIP_OK;
}

// Host-side range checks on host-resident block_table / context_lens
// (the reference's orchestration reads both on the host side as well,
// paged_attention_orch.cpp:165-180).
int check_host_tables(const SimplerChipStorageTaskArgs *a, const SimplerHipPaDecodeArgs &pa) {
    const SimplerChipTensor &bt = tensor_at(a, 3), &cl = tensor_at(a, 4);
    if (bt.address_space != SIMPLER_ADDR_HOST || cl.address_space != SIMPLER_ADDR_HOST) return SIMPLER_HIP_OK;
    const int32_t *lens = (const int32_t *)(uintptr_t)cl.buffer.addr + cl.start_offset;
    const int32_t *tab = (const int32_t *)(uintptr_t)bt.buffer.addr + bt.start_offset;
    for (int b = 0; b < pa.batch; ++b) {
        const int64_t len = lens[b];
        if (len < 0 || len > (int64_t)pa.max_blocks_per_seq * pa.block_size) {
            logf("context_lens[%d] = %lld outside [0, %lld]", b, (long long)len,
                 (long long)pa.max_blocks_per_seq * pa.block_size);
            return SIMPLER_HIP_ERR_INVALID;
        }
        if (pa.causal && len < pa.q_len) {
            logf("context_lens[%d] = %lld shorter than q_len %d", b, (long long)len, pa.q_len);
            return SIMPLER_HIP_ERR_INVALID;
        }
        const int nblk = (int)((len + pa.block_size - 1) / pa.block_size);
        for (int j = 0; j < nblk; ++j) {
            const int32_t e = tab[(int64_t)b * pa.max_blocks_per_seq + j];
            if (e < 0 || e >= pa.num_blocks) {
                logf("block_table[%d][%d] = %d outside the pool of %d blocks", b, j, e, pa.num_blocks);
                return SIMPLER_HIP_ERR_INVALID;
            }
        }
    }
    return SIMPLER_HIP_OK;
}

int ensure_workspace(DeviceContext *c, size_t need) {
    if (need <= c->workspace_bytes) return SIMPLER_HIP_OK;
    if (c->workspace) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(c->workspace);
        c->workspace = nullptr;
        c->workspace_bytes = 0;
    }
    size_t sz = need < (1u << 20) ? (1u << 20) : need;
    if (hipMalloc(&c->workspace, sz) != hipSuccess) {
        logf("workspace allocation of %zu bytes failed", sz);
        c->workspace = nullptr;
        return SIMPLER_HIP_ERR_WORKSPACE;
    }
    c->workspace_bytes = sz;
    return simpler_hip_pa_decode_workspace_init(c->workspace, sz, c->stream);
}

int check_vector_args(const SimplerChipStorageTaskArgs *a) {
    if (a->tensor_count_ < kVecTensors) {
        logf("vector example needs 3 tensors (a, b, f)");
        return SIMPLER_HIP_ERR_INVALID;
    }
    const SimplerChipTensor &x = tensor_at(a, 0);
    for (int i = 0; i < kVecTensors; ++i) {
        const SimplerChipTensor &t = tensor_at(a, i);
        if (t.dtype != SIMPLER_DT_FLOAT32 || t.ndims != 1 || t.shapes[0] != x.shapes[0] || !contiguous(t)) {
            logf("vector example tensors must be contiguous fp32 [n] of one size");
            return SIMPLER_HIP_ERR_INVALID;
        }
    }
    return SIMPLER_HIP_OK;
}

// Runs the callable's orchestration on the context's task graph for the
// run's execution mode (eager launches, or one hipGraph launched at the end).
int run_task_graph(DeviceContext *c, NativeRun *r) {
    const int slot = r->execution == SIMPLER_HIP_EXEC_TASK_GRAPH_HIPGRAPH ? 1 : 0;
    SimplerHipTaskGraph *&g = c->graphs[slot];
    if (!g) {
        g = simpler_hip_tg_create(slot ? SIMPLER_HIP_TG_GRAPH : SIMPLER_HIP_TG_EAGER, c->stream);
        if (!g) return SIMPLER_HIP_ERR_LAUNCH;
    }
    int rc = simpler_hip_tg_reset(g);
    if (rc != SIMPLER_HIP_OK) return rc;
    simpler_hip_tg_scope_begin(g);  // the executor's outer scope
    rc = r->kind == kPagedAttention ? simpler_hip_tg_orchestrate_paged_attention(g, r->tensors, r->scale_bits)
                                    : simpler_hip_tg_orchestrate_vector_example(g, r->tensors);
    if (rc != SIMPLER_HIP_OK) {
        simpler_hip_tg_reset(g);
        return rc;
    }
    simpler_hip_tg_scope_end(g);
    return simpler_hip_tg_launch(g);
}

void release_staged(NativeRun *r) {
    for (int i = 0; i < r->n_staged; ++i) {
        if (r->staged_dev[i]) (void)hipFree(r->staged_dev[i]);
        r->staged_dev[i] = nullptr;
    }
    r->n_staged = 0;
    free(r->host_lens);
    r->host_lens = nullptr;
}

// Tiling-tensor layout of the high-performance SPMD callable
// (tests/st/.../spmd_paged_attention_highperf/kernels/pa_tiling.py:18-62,360-430):
// a header of TILING_HEAD_SIZE int32 words, then TILING_PARA_SIZE words per
// sequence, word 1 of which is the sequence's KV length.
constexpr int kTilingBatch = 0, kTilingNumHeads = 1, kTilingHeadDim = 2, kTilingBlockSize = 4, kTilingTor = 6,
              kTilingKvHeads = 7, kTilingHeadSize = 17, kTilingParaSize = 18, kTilingParaKvSeqLen = 1;
constexpr int kTilingMinHeader = 19;

// Rewrites the high-performance callable's arguments into the common 7-argument
// form (query, key_cache, value_cache, block_table, context_lens, out; scale):
// the lengths and the scale come from the tiling tensor (tensor 13), read on
// the host (copied back first when it is device-resident); the workspaces
// (tensors 5..12) and tensor 14 are not used. r->host_lens keeps the lengths
// until the run is finalised.
int remap_highperf(const SimplerChipStorageTaskArgs *a, NativeRun *r, SimplerChipStorageTaskArgs *out) {
    if (a->tensor_count_ < kHighperfTensors) {
        logf("the high-performance paged-attention callable takes %d tensors (got %d)", kHighperfTensors,
             a->tensor_count_);
        return SIMPLER_HIP_ERR_INVALID;
    }
    const SimplerChipTensor &q = tensor_at(a, 0), &k = tensor_at(a, 1), &tl = tensor_at(a, 13);
    uint64_t n = 1;
    for (uint32_t d = 0; d < tl.ndims; ++d) n *= tl.shapes[d];
    if (tl.dtype != SIMPLER_DT_INT32 || !contiguous(tl) || n < kTilingMinHeader || n > (1u << 26)) {
        logf("tiling must be a contiguous INT32 tensor with a header");
        return SIMPLER_HIP_ERR_INVALID;
    }
    std::vector<int32_t> w(n);
    const void *src = (const void *)(uintptr_t)(tl.buffer.addr + tl.start_offset * 4);
    if (tl.address_space == SIMPLER_ADDR_DEVICE) {
        if (hipMemcpy(w.data(), src, n * 4, hipMemcpyDeviceToHost) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    } else {
        memcpy(w.data(), src, n * 4);
    }
    const int64_t batch = w[kTilingBatch], head = w[kTilingHeadSize], para = w[kTilingParaSize];
    if (q.ndims != 3 || k.ndims != 4 || batch != (int64_t)q.shapes[0] || w[kTilingNumHeads] != (int32_t)q.shapes[1] ||
        w[kTilingHeadDim] != (int32_t)q.shapes[2] || w[kTilingBlockSize] != (int32_t)k.shapes[1] ||
        w[kTilingKvHeads] != (int32_t)k.shapes[2] || head < kTilingMinHeader || para < kTilingParaKvSeqLen + 1 ||
        (uint64_t)(head + batch * para) > n) {
        logf("tiling header disagrees with the query [B, Hq, D] / key_cache [nblk, BS, Hkv, D] shapes");
        return SIMPLER_HIP_ERR_INVALID;
    }
    r->host_lens = static_cast<int32_t *>(malloc((size_t)(batch > 0 ? batch : 1) * 4));
    if (!r->host_lens) return SIMPLER_HIP_ERR_WORKSPACE;
    for (int64_t b = 0; b < batch; ++b) r->host_lens[b] = w[head + b * para + kTilingParaKvSeqLen];
    memset(out, 0, sizeof(*out));
    for (int i = 0; i < 4; ++i) out->tensors_[i] = a->tensors_[i];
    SimplerChipTensor &cl = out->tensors_[4];
    cl.buffer.addr = (uint64_t)(uintptr_t)r->host_lens;
    cl.buffer.size = (uint64_t)batch * 4;
    cl.ndims = 1;
    cl.shapes[0] = (uint32_t)batch;
    cl.strides[0] = 1;
    cl.dtype = SIMPLER_DT_INT32;
    cl.is_contiguous = 1;
    cl.address_space = SIMPLER_ADDR_HOST;
    cl.extent_elem_cache = (uint64_t)batch;
    out->tensors_[5] = a->tensors_[4];
    out->tensor_count_ = kPaTensors;
    out->scalars_[0] = (uint32_t)w[kTilingTor];  // the scale, as fp32 bits
    out->scalar_count_ = 1;
    return SIMPLER_HIP_OK;
}

}  // namespace

extern "C" {

const PipelineContract *get_pipeline_contract(void) { return &kContract; }
size_t get_runtime_size(void) { return (sizeof(NativeRun) + 255) / 256 * 256; }
size_t get_runtime_alignment(void) { return 64; }

DeviceContextHandle create_device_context(void) { return new (std::nothrow) DeviceContext(); }

void destroy_device_context(DeviceContextHandle h) {
    DeviceContext *c = as_ctx(h);
    if (!c) return;
    finalize_device(h);
    delete c;
}

int simpler_init(DeviceContextHandle h, int device_id, const uint8_t *, size_t, const uint8_t *, size_t,
                 const uint8_t *, size_t, const struct CallConfig *) {
    DeviceContext *c = as_ctx(h);
    if (!c) return -1;
    std::lock_guard<std::mutex> lk(c->mu);
    if (c->device_id >= 0) return c->device_id == device_id ? 0 : -1;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device_id < 0 || device_id >= n) {
        logf("no HIP device %d (devices visible: %d)", device_id, n);
        return -1;
    }
    if (hipSetDevice(device_id) != hipSuccess) return -1;
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return -1;
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipStreamDestroy(s);
        return -1;
    }
    void *pinned = nullptr;
    if (hipHostMalloc(&pinned, 64, hipHostMallocCoherent) != hipSuccess) {
        (void)hipEventDestroy(ev);
        (void)hipStreamDestroy(s);
        return -1;
    }
    *static_cast<unsigned *>(pinned) = 0;
    c->device_id = device_id;
    c->stream = s;
    c->done = ev;
    c->err_host = static_cast<unsigned *>(pinned);
    if (const char *e = getenv("SIMPLER_HIP_EXECUTION")) {
        if (strcmp(e, "eager") == 0) c->execution = SIMPLER_HIP_EXEC_TASK_GRAPH;
        else if (strcmp(e, "graph") == 0) c->execution = SIMPLER_HIP_EXEC_TASK_GRAPH_HIPGRAPH;
    }
    return 0;
}

int finalize_device(DeviceContextHandle h) {
    DeviceContext *c = as_ctx(h);
    if (!c) return -1;
    std::lock_guard<std::mutex> lk(c->mu);
    if (c->device_id < 0) return 0;
    (void)hipSetDevice(c->device_id);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (SimplerHipTaskGraph *&g : c->graphs) {
        simpler_hip_tg_destroy(g);
        g = nullptr;
    }
    for (auto &kv : c->allocs) (void)hipFree(kv.first);
    c->allocs.clear();
    c->committed = 0;
    if (c->workspace) (void)hipFree(c->workspace);
    c->workspace = nullptr;
    c->workspace_bytes = 0;
    if (c->done) (void)hipEventDestroy(c->done);
    c->done = nullptr;
    if (c->err_host) (void)hipHostFree(c->err_host);
    c->err_host = nullptr;
    if (c->stream) (void)hipStreamDestroy(c->stream);
    c->stream = nullptr;
    c->device_id = -1;
    return 0;
}

void *device_malloc_ctx(DeviceContextHandle h, size_t size) {
    DeviceContext *c = as_ctx(h);
    if (!set_device(c)) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, size ? size : 1) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(c->mu);
    c->allocs[p] = size;
    c->committed += size;
    return p;
}

void device_free_ctx(DeviceContextHandle h, void *p) {
    DeviceContext *c = as_ctx(h);
    if (!set_device(c) || !p) return;
    std::lock_guard<std::mutex> lk(c->mu);
    auto it = c->allocs.find(p);
    if (it == c->allocs.end()) return;
    (void)hipStreamSynchronize(c->stream);
    c->committed -= it->second;
    c->allocs.erase(it);
    (void)hipFree(p);
}

size_t committed_device_memory_ctx(DeviceContextHandle h) {
    DeviceContext *c = as_ctx(h);
    if (!c) return 0;
    std::lock_guard<std::mutex> lk(c->mu);
    return c->committed;
}

int copy_to_device_ctx(DeviceContextHandle h, void *dev, const void *host, size_t size) {
    DeviceContext *c = as_ctx(h);
    if (!set_device(c)) return -1;
    if (hipMemcpyAsync(dev, host, size, hipMemcpyHostToDevice, c->stream) != hipSuccess) return -1;
    return hipStreamSynchronize(c->stream) == hipSuccess ? 0 : -1;
}

int copy_from_device_ctx(DeviceContextHandle h, void *host, const void *dev, size_t size) {
    DeviceContext *c = as_ctx(h);
    if (!set_device(c)) return -1;
    if (hipMemcpyAsync(host, dev, size, hipMemcpyDeviceToHost, c->stream) != hipSuccess) return -1;
    return hipStreamSynchronize(c->stream) == hipSuccess ? 0 : -1;
}

int simpler_register_callable(DeviceContextHandle h, int32_t id, const void *callable) {
    DeviceContext *c = as_ctx(h);
    if (!c || !callable || id < 0 || id >= kMaxCallables) return -1;
    Callable cb;
    const CallableKind kind = classify(static_cast<const uint8_t *>(callable), cb);
    if (kind == kNone) {
        logf("callable %d is neither the paged-attention chain nor the vector example; the HIP backend runs those",
             id);
        return PTO_RUNTIME_ERR_UNSUPPORTED;
    }
    cb.kind = kind;
    std::lock_guard<std::mutex> lk(c->mu);
    c->callables[id] = cb;
    return 0;
}

int simpler_unregister_callable(DeviceContextHandle h, int32_t id) {
    DeviceContext *c = as_ctx(h);
    if (!c || id < 0 || id >= kMaxCallables) return -1;
    std::lock_guard<std::mutex> lk(c->mu);
    c->callables[id] = Callable();
    return 0;
}

int supports_concurrent_native_prepare_ctx(DeviceContextHandle) { return 0; }

int simpler_prepare_run(DeviceContextHandle h, RuntimeHandle runtime, int32_t id, const void *args_v,
                        const struct CallConfig *, const NativeRunDescriptor *) {
    DeviceContext *c = as_ctx(h);
    NativeRun *r = static_cast<NativeRun *>(runtime);
    if (!set_device(c) || !r || !args_v || id < 0 || id >= kMaxCallables) return -1;
    if (r->magic == kRunMagic && r->state != 0) return PTO_RUNTIME_ERR_PREPARED_INCOMPATIBLE;
    Callable cb;
    int32_t execution;
    {
        std::lock_guard<std::mutex> lk(c->mu);
        cb = c->callables[id];
        execution = c->execution;
    }
    if (cb.kind == kNone) {
        logf("callable %d is not registered", id);
        return -1;
    }
    // The POD is 64-byte aligned in C++; callers from other languages may hand
    // over less-aligned storage, so decode from an aligned copy.
    std::unique_ptr<SimplerChipStorageTaskArgs> aligned_copy;
    const SimplerChipStorageTaskArgs *a = static_cast<const SimplerChipStorageTaskArgs *>(args_v);
    if ((uintptr_t)args_v % alignof(SimplerChipStorageTaskArgs)) {
        aligned_copy.reset(new (std::nothrow) SimplerChipStorageTaskArgs);
        if (!aligned_copy) return SIMPLER_HIP_ERR_WORKSPACE;
        memcpy(aligned_copy.get(), args_v, sizeof(SimplerChipStorageTaskArgs));
        a = aligned_copy.get();
    }
    memset(r, 0, sizeof(*r));
    r->magic = kRunMagic;
    r->callable_id = id;
    r->kind = cb.kind;
    r->execution = cb.kind == kVectorExample && execution == SIMPLER_HIP_EXEC_FUSED ? SIMPLER_HIP_EXEC_TASK_GRAPH
                                                                                    : execution;
    int rc = SIMPLER_HIP_OK;
    // The high-performance callable's arguments, rewritten into the common form
    std::unique_ptr<SimplerChipStorageTaskArgs> remapped;
    if (cb.kind == kPagedAttention && cb.family == kPaHighperf) {
        remapped.reset(new (std::nothrow) SimplerChipStorageTaskArgs);
        if (!remapped) rc = SIMPLER_HIP_ERR_WORKSPACE;
        if (rc == SIMPLER_HIP_OK) rc = remap_highperf(a, r, remapped.get());
        if (rc != SIMPLER_HIP_OK) {
            release_staged(r);
            r->magic = 0;
            return rc;
        }
        a = remapped.get();
    }
    if (cb.kind == kPagedAttention) {
        r->n_tensors = kPaTensors;
        rc = decode_pa_args(a, r->args, cb.family == kPaHighperf ? kMaxRunTensors : 1);
        if (rc == SIMPLER_HIP_OK && r->args.kv_format == SIMPLER_HIP_KV_FP8_E4M3) r->n_tensors = kPaTensors + 2;
        if (rc == SIMPLER_HIP_OK) rc = check_host_tables(a, r->args);
        if (rc == SIMPLER_HIP_OK && r->execution != SIMPLER_HIP_EXEC_FUSED &&
            (r->args.num_kv_heads != 1 || r->args.q_len != 1 || r->args.head_dim_k != r->args.head_dim_v ||
             r->args.kv_format != SIMPLER_HIP_KV_BF16)) {
            logf("task-graph paged attention runs the reference orchestration: one KV head, one query token, "
                 "Dk == Dv, bf16 caches");
            rc = SIMPLER_HIP_ERR_UNSUPPORTED;
        }
        if (rc == SIMPLER_HIP_OK && r->execution != SIMPLER_HIP_EXEC_FUSED && cb.family != kPaChain &&
            cb.family != kPaNative) {  // also the highperf family
            logf("the task-graph backend runs the per-block QK/SF/PV/UP orchestration only; the grouped and "
                 "SPMD paged-attention callables run on the fused kernel");
            rc = SIMPLER_HIP_ERR_UNSUPPORTED;
        }
        r->scale_bits = a->scalars_[0];
    } else {
        r->n_tensors = kVecTensors;
        rc = check_vector_args(a);
    }
    if (rc != SIMPLER_HIP_OK) {
        release_staged(r);
        r->magic = 0;
        return rc;
    }
    // Stage host tensors; directions from the callable signature (for the
    // rewritten high-performance arguments, those of the common form).
    const void *dev[kMaxRunTensors];
    for (int i = 0; i < r->n_tensors; ++i) {
        const SimplerChipTensor &t = tensor_at(a, i);
        const size_t esz = simpler_dtype_size(t.dtype);
        const int dir = remapped ? kOrchSig[i] : (i < cb.sig_count ? cb.sig[i] : SIMPLER_ARG_IN);
        r->tensors[i] = t;
        if (t.address_space == SIMPLER_ADDR_DEVICE) {
            dev[i] = (const void *)(uintptr_t)(t.buffer.addr + t.start_offset * esz);
            continue;
        }
        // Tables the task-graph orchestration only reads on the host stay there.
        if (cb.kind == kPagedAttention && r->execution != SIMPLER_HIP_EXEC_FUSED && (i == 3 || i == 4)) {
            dev[i] = nullptr;
            continue;
        }
        const size_t bytes = extent_bytes(t);
        void *d = nullptr;
        if (hipMalloc(&d, bytes ? bytes : 1) != hipSuccess) {
            logf("staging allocation of %zu bytes failed", bytes);
            release_staged(r);
            r->magic = 0;
            return SIMPLER_HIP_ERR_WORKSPACE;
        }
        const int slot = r->n_staged++;
        r->staged_dev[slot] = d;
        r->host_ptr[slot] = (void *)(uintptr_t)t.buffer.addr;
        r->staged_bytes[slot] = bytes;
        r->dir[slot] = dir;
        if (dir != SIMPLER_ARG_OUT &&
            hipMemcpyAsync(d, (const void *)(uintptr_t)t.buffer.addr, bytes, hipMemcpyHostToDevice, c->stream) !=
                hipSuccess) {
            release_staged(r);
            r->magic = 0;
            return SIMPLER_HIP_ERR_LAUNCH;
        }
        dev[i] = (const char *)d + t.start_offset * esz;
        r->tensors[i].buffer.addr = (uint64_t)(uintptr_t)d;
        r->tensors[i].buffer.size = bytes;
        r->tensors[i].address_space = SIMPLER_ADDR_DEVICE;
    }
    if (cb.kind == kPagedAttention && r->execution == SIMPLER_HIP_EXEC_FUSED) {
        r->args.query = dev[0];
        r->args.key_cache = dev[1];
        r->args.value_cache = dev[2];
        r->args.block_table = (const int32_t *)dev[3];
        r->args.context_lens = (const int32_t *)dev[4];
        r->args.out = (void *)dev[5];
        if (r->args.kv_format == SIMPLER_HIP_KV_FP8_E4M3) {
            r->args.k_scale = (const float *)dev[6];
            r->args.v_scale = (const float *)dev[7];
        }
        const size_t need = simpler_hip_pa_decode_workspace_size(&r->args);
        if (need == 0) {
            release_staged(r);
            r->magic = 0;
            return SIMPLER_HIP_ERR_INVALID;
        }
        {
            std::lock_guard<std::mutex> lk(c->mu);
            rc = ensure_workspace(c, need);
        }
        if (rc != SIMPLER_HIP_OK) {
            release_staged(r);
            r->magic = 0;
            return rc;
        }
    }
    r->done = c->done;
    r->state = 1;
    return 0;
}

int simpler_launch_run(DeviceContextHandle h, RuntimeHandle runtime) {
    DeviceContext *c = as_ctx(h);
    NativeRun *r = static_cast<NativeRun *>(runtime);
    if (!set_device(c) || !r || r->magic != kRunMagic || r->state != 1) return -1;
    int rc;
    if (r->kind == kPagedAttention && r->execution == SIMPLER_HIP_EXEC_FUSED) {
        // the merge kernel overwrites it; a batch of 0 launches nothing
        __atomic_store_n(c->err_host, 0u, __ATOMIC_RELEASE);
        rc = simpler_hip::pa_decode_with_mirror(&r->args, c->workspace, c->workspace_bytes, c->stream, c->err_host);
    } else {
        rc = run_task_graph(c, r);
    }
    if (rc != SIMPLER_HIP_OK) return rc;
    for (int i = 0; i < r->n_staged; ++i) {
        if (r->dir[i] == SIMPLER_ARG_IN) continue;
        if (hipMemcpyAsync(r->host_ptr[i], r->staged_dev[i], r->staged_bytes[i], hipMemcpyDeviceToHost,
                           c->stream) != hipSuccess)
            return SIMPLER_HIP_ERR_LAUNCH;
    }
    if (hipEventRecord(r->done, c->stream) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    r->state = 2;
    ++c->runs;
    return 0;
}

int simpler_poll_run(DeviceContextHandle h, RuntimeHandle runtime) {
    DeviceContext *c = as_ctx(h);
    NativeRun *r = static_cast<NativeRun *>(runtime);
    if (!set_device(c) || !r || r->magic != kRunMagic || r->state != 2) return SIMPLER_NATIVE_RUN_POLL_ERROR;
    const hipError_t e = hipEventQuery(r->done);
    if (e == hipSuccess) return SIMPLER_NATIVE_RUN_POLL_COMPLETE;
    if (e == hipErrorNotReady) return SIMPLER_NATIVE_RUN_POLL_NOT_READY;
    return SIMPLER_NATIVE_RUN_POLL_ERROR;
}

int simpler_wait_run(DeviceContextHandle h, RuntimeHandle runtime) {
    DeviceContext *c = as_ctx(h);
    NativeRun *r = static_cast<NativeRun *>(runtime);
    if (!set_device(c) || !r || r->magic != kRunMagic || r->state != 2) return -1;
    if (hipEventSynchronize(r->done) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    if (r->kind != kPagedAttention || r->execution != SIMPLER_HIP_EXEC_FUSED) return SIMPLER_HIP_OK;
    if (__atomic_load_n(c->err_host, __ATOMIC_ACQUIRE) == 0) return SIMPLER_HIP_OK;
    // A bad block id was seen: the check re-reads the device word and clears it.
    return simpler_hip_pa_decode_check(c->workspace, c->workspace_bytes, c->stream);
}

int simpler_finalize_run(DeviceContextHandle h, RuntimeHandle runtime) {
    DeviceContext *c = as_ctx(h);
    NativeRun *r = static_cast<NativeRun *>(runtime);
    if (!set_device(c) || !r) return -1;
    if (r->magic != kRunMagic) return 0;
    if (r->state == 2) (void)hipEventSynchronize(r->done);
    release_staged(r);
    memset(r, 0, sizeof(*r));
    return 0;
}

int simpler_run(DeviceContextHandle h, RuntimeHandle runtime, int32_t id, const void *args,
                const struct CallConfig *config, const NativeRunDescriptor *desc) {
    int rc = simpler_prepare_run(h, runtime, id, args, config, desc);
    if (rc != 0) return rc;
    rc = simpler_launch_run(h, runtime);
    int rc2 = rc == 0 ? simpler_wait_run(h, runtime) : rc;
    simpler_finalize_run(h, runtime);
    return rc2;
}

uint64_t get_arena_bank_gm_heap_base_ctx(DeviceContextHandle, uint32_t) { return 0; }
uint64_t get_retained_temp_addr_ctx(DeviceContextHandle, uint32_t) { return 0; }
size_t get_aicpu_dlopen_count(DeviceContextHandle) { return 0; }
size_t get_host_dlopen_count(DeviceContextHandle) { return 0; }
size_t get_run_stream_set_create_count(DeviceContextHandle h) { return as_ctx(h) && as_ctx(h)->stream ? 1 : 0; }
int simpler_provision_dma_workspace(DeviceContextHandle, uint32_t required_mask, const void *, uint64_t) {
    return required_mask == 0 ? 0 : PTO_RUNTIME_ERR_UNSUPPORTED;
}

int ensure_acl_ready_ctx(DeviceContextHandle, int) { return PTO_RUNTIME_ERR_UNSUPPORTED; }
void *create_comm_stream_ctx(DeviceContextHandle) { return nullptr; }
int destroy_comm_stream_ctx(DeviceContextHandle, void *) { return PTO_RUNTIME_ERR_UNSUPPORTED; }

CommHandle comm_init(int, int, void *, const char *) { return nullptr; }
int comm_alloc_windows(CommHandle, size_t, uint64_t *) { return PTO_RUNTIME_ERR_UNSUPPORTED; }
int comm_get_local_window_base(CommHandle, uint64_t *) { return PTO_RUNTIME_ERR_UNSUPPORTED; }
int comm_get_window_size(CommHandle, size_t *) { return PTO_RUNTIME_ERR_UNSUPPORTED; }
int comm_derive_context(CommHandle, const uint32_t *, size_t, uint32_t, size_t, size_t, uint64_t *) {
    return PTO_RUNTIME_ERR_UNSUPPORTED;
}
int comm_alloc_domain_windows(CommHandle, uint64_t, const uint32_t *, size_t, uint32_t, size_t, uint64_t *,
                              uint64_t *) {
    return PTO_RUNTIME_ERR_UNSUPPORTED;
}
int comm_release_domain_windows(CommHandle, uint64_t, size_t, uint32_t) { return PTO_RUNTIME_ERR_UNSUPPORTED; }
int comm_global_domain_prepare(uint64_t, uint32_t, uint32_t, size_t, uint32_t, CommGlobalDomainDescriptor *,
                               uint64_t *) {
    return PTO_RUNTIME_ERR_UNSUPPORTED;
}
int comm_global_domain_import(uint64_t, const CommGlobalDomainDescriptor *, size_t, uint64_t *) {
    return PTO_RUNTIME_ERR_UNSUPPORTED;
}
int comm_global_domain_release(uint64_t) { return PTO_RUNTIME_ERR_UNSUPPORTED; }
int comm_barrier(CommHandle) { return PTO_RUNTIME_ERR_UNSUPPORTED; }
int comm_destroy(CommHandle) { return PTO_RUNTIME_ERR_UNSUPPORTED; }

void *simpler_hip_context_stream(DeviceContextHandle h) { return as_ctx(h) ? (void *)as_ctx(h)->stream : nullptr; }

int simpler_hip_callable_family(DeviceContextHandle h, int32_t id) {
    DeviceContext *c = as_ctx(h);
    if (!c || id < 0 || id >= kMaxCallables) return -1;
    std::lock_guard<std::mutex> lk(c->mu);
    return c->callables[id].kind == kPagedAttention ? c->callables[id].family : -1;
}

int simpler_hip_set_execution(DeviceContextHandle h, int32_t execution) {
    DeviceContext *c = as_ctx(h);
    if (!c || execution < SIMPLER_HIP_EXEC_FUSED || execution > SIMPLER_HIP_EXEC_TASK_GRAPH_HIPGRAPH) return -1;
    std::lock_guard<std::mutex> lk(c->mu);
    c->execution = execution;
    return 0;
}

}  // extern "C"
