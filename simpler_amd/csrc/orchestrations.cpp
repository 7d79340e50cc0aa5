// Orchestrations for the task-graph backend: the reference examples'
// aicpu_orchestration_entry functions, rewritten against the task-graph C API
// and run on the host (the host-build-graph style: the submits are recorded,
// dependencies inferred, kernels launched on the device).
//
//   simpler_hip_tg_orchestrate_paged_attention
//     <- examples/a2a3/tensormap_and_ringbuffer/paged_attention/kernels/orchestration/paged_attention_orch.cpp:77-249
//   simpler_hip_tg_orchestrate_vector_example
//     <- examples/a2a3/tensormap_and_ringbuffer/vector_example/kernels/orchestration/example_orchestration.cpp:55-112
//
// The small Args / view / create-info helpers below have the roles of the
// reference's CoreTaskArgs (runtime/pto_types.h:374-398), ChipTensor::view
// (src/common/task_interface/tensor.h:283-312), make_tensor_external
// (tensor.h:509-518) and TensorCreateInfo.

#include <algorithm>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <vector>

#include "simpler_hip/task_graph.h"
#include "task_graph_internal.h"

namespace {

void orch_log(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "[simpler_hip orchestration] ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
}

SimplerChipTensor create_info(const uint32_t *shapes, uint32_t ndims, uint8_t dtype) {
    SimplerChipTensor t;
    memset(&t, 0, sizeof(t));
    t.ndims = ndims;
    t.dtype = dtype;
    uint64_t acc = 1;
    for (int d = (int)ndims - 1; d >= 0; --d) {
        t.shapes[d] = shapes[d];
        t.strides[d] = (uint32_t)acc;
        acc *= shapes[d];
    }
    t.owner_task_id = SIMPLER_HIP_TASK_INVALID;
    return t;
}

// Row-major tensor over existing device memory, no producer.
SimplerChipTensor external(uint64_t addr, const uint32_t *shapes, uint32_t ndims, uint8_t dtype) {
    SimplerChipTensor t = create_info(shapes, ndims, dtype);
    t.buffer.addr = addr;
    uint64_t n = 1;
    for (uint32_t d = 0; d < ndims; ++d) n *= shapes[d];
    t.buffer.size = n * simpler_dtype_size(dtype);
    t.is_contiguous = 1;
    t.address_space = SIMPLER_ADDR_DEVICE;
    t.extent_elem_cache = n;
    return t;
}

SimplerChipTensor view(const SimplerChipTensor &src, const uint32_t *shapes, const uint32_t *offsets) {
    SimplerChipTensor t = src;
    for (uint32_t d = 0; d < src.ndims; ++d) {
        t.start_offset += (uint64_t)offsets[d] * src.strides[d];
        t.shapes[d] = shapes[d];
    }
    return t;
}

struct Args {
    SimplerChipTensor t[SIMPLER_CORE_MAX_TENSOR_ARGS];
    int32_t tag[SIMPLER_CORE_MAX_TENSOR_ARGS];
    uint64_t s[SIMPLER_CORE_MAX_SCALAR_ARGS];
    int32_t n = 0, ns = 0;
    void add(const SimplerChipTensor &x, int32_t ty) {
        t[n] = x;
        tag[n++] = ty;
    }
    void add_input(const SimplerChipTensor &x) { add(x, SIMPLER_HIP_TA_INPUT); }
    void add_output(const SimplerChipTensor &ci) { add(ci, SIMPLER_HIP_TA_OUTPUT); }
    void add_output_existing(const SimplerChipTensor &x) { add(x, SIMPLER_HIP_TA_OUTPUT_EXISTING); }
    void add_inout(const SimplerChipTensor &x) { add(x, SIMPLER_HIP_TA_INOUT); }
    void add_scalar(uint64_t v) { s[ns++] = v; }
};

// Submits and returns the runtime-created outputs in add order
// (TaskOutputTensors::get_ref).
struct Submitted {
    int64_t task = -1;
    SimplerChipTensor out[SIMPLER_CORE_MAX_TENSOR_ARGS];
    int32_t n_out = 0;
};

Submitted submit(SimplerHipTaskGraph *g, int32_t func_id, const Args &a) {
    Submitted r;
    SimplerChipTensor all[SIMPLER_CORE_MAX_TENSOR_ARGS];
    r.task = simpler_hip_tg_submit(g, func_id, a.t, a.tag, a.n, a.s, a.ns, nullptr, 0, all);
    if (r.task < 0) return r;
    for (int i = 0; i < a.n; ++i)
        if (a.tag[i] == SIMPLER_HIP_TA_OUTPUT) r.out[r.n_out++] = all[i];
    return r;
}

// Replay key of a step: bytes appended in the order the orchestration reads them.
struct StepKey {
    std::vector<uint8_t> bytes;
    void add(const void *p, size_t n) {
        const uint8_t *b = static_cast<const uint8_t *>(p);
        bytes.insert(bytes.end(), b, b + n);
    }
    void add_u64(uint64_t v) { add(&v, sizeof(v)); }
};

// A step replays in GRAPH mode only (there the host's orchestration is the
// step's critical path; elsewhere the key's table reads would be wasted), and
// only when it starts on a reset graph, so that its key describes every task
// the graph will hold.
bool replayable(const SimplerHipTaskGraph *g) {
    return simpler_hip::tg_mode_of(g) == SIMPLER_HIP_TG_GRAPH && simpler_hip::tg_is_fresh(g);
}

uint64_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

constexpr int32_t FUNC_QK_MATMUL = 0, FUNC_SOFTMAX_PREPARE = 1, FUNC_PV_MATMUL = 2, FUNC_ONLINE_UPDATE = 3;
// Not a reference func id: the zero output of an empty context (see below).
constexpr int32_t FUNC_ZERO_FILL = 4;

}  // namespace

extern "C" {

int simpler_hip_tg_orchestrate_paged_attention(SimplerHipTaskGraph *g, const SimplerChipTensor *tensors,
                                               uint64_t scale_bits) {
    if (!g || !tensors) return SIMPLER_HIP_ERR_INVALID;
    const SimplerChipTensor &q = tensors[0], &kc = tensors[1], &vc = tensors[2], &bt = tensors[3],
                            &cl = tensors[4], &o = tensors[5];
    // shapes as the reference reads them (paged_attention_orch.cpp:94-102)
    if (q.ndims != 3 || (kc.ndims != 3 && kc.ndims != 4) || kc.ndims != vc.ndims || bt.ndims != 2 ||
        cl.ndims != 1 || (o.ndims != 3 && o.ndims != 2)) {
        orch_log("paged attention: query [B,Hq,D], caches [nblk,BS,(1,)D], block_table [B,maxblk], "
                 "context_lens [B], out [B,Hq,D]");
        return SIMPLER_HIP_ERR_INVALID;
    }
    const uint32_t batch = q.shapes[0], num_heads = q.shapes[1], head_dim = q.shapes[2];
    const uint32_t block_size = kc.shapes[1], block_num = bt.shapes[1], total_blocks = kc.shapes[0];
    // The reference flattens the caches to [nblk*BS, D] (:119-126), which is
    // only meaningful for one KV head.
    if (kc.ndims == 4 && (kc.shapes[2] != 1 || vc.shapes[2] != 1)) {
        orch_log("paged attention (task graph): one KV head only, as the reference orchestration");
        return SIMPLER_HIP_ERR_UNSUPPORTED;
    }
    if (kc.shapes[kc.ndims - 1] != head_dim || vc.shapes[vc.ndims - 1] != head_dim || vc.shapes[0] != total_blocks ||
        vc.shapes[1] != block_size || bt.shapes[0] != batch || cl.shapes[0] != batch ||
        q.dtype != SIMPLER_DT_BFLOAT16 || kc.dtype != q.dtype || vc.dtype != q.dtype ||
        bt.dtype != SIMPLER_DT_INT32 || cl.dtype != SIMPLER_DT_INT32 ||
        (o.dtype != SIMPLER_DT_FLOAT32 && o.dtype != SIMPLER_DT_BFLOAT16)) {
        orch_log("paged attention (task graph): shapes or dtypes disagree");
        return SIMPLER_HIP_ERR_INVALID;
    }
    for (int32_t f = 0; f < 4; ++f) simpler_hip_tg_bind(g, f, f);  // FUNC_* ids equal the kernel codes
    simpler_hip_tg_bind(g, FUNC_ZERO_FILL, SIMPLER_HIP_K_ZERO_FILL);

    // GRAPH mode: the step is a function of the six tensors, the scale and
    // the table values read below (context_lens[b], then block_table[b][bn]
    // for the blocks it covers). With the same key as the recorded step, the
    // recorded DAG is restored instead of being orchestrated again.
    StepKey key;
    const bool replay = replayable(g);
    if (replay) {
        const SimplerChipTensor tables[2] = {cl, bt};
        int rc = simpler_hip::tg_prefetch_host(g, tables, 2);  // both tables, one synchronisation
        if (rc != SIMPLER_HIP_OK) return rc;
        key.add(tensors, 6 * sizeof(SimplerChipTensor));
        key.add_u64(scale_bits);
        for (uint32_t b = 0; b < batch; ++b) {
            uint64_t raw = 0;
            const uint32_t cl_idx[1] = {b};
            rc = simpler_hip_tg_get_tensor_data(g, &cl, 1, cl_idx, &raw);
            if (rc != SIMPLER_HIP_OK) return rc;
            key.add_u64(raw);
            const int64_t len = (int32_t)(uint32_t)raw;
            const uint64_t nb = len <= 0 ? 0 : std::min<uint64_t>(((uint64_t)len + block_size - 1) / block_size, block_num);
            for (uint64_t bn = 0; bn < nb; ++bn) {
                const uint32_t bt_idx[2] = {b, (uint32_t)bn};
                rc = simpler_hip_tg_get_tensor_data(g, &bt, 2, bt_idx, &raw);
                if (rc != SIMPLER_HIP_OK) return rc;
                key.add_u64(raw);
            }
        }
        if (simpler_hip_tg_replay(g, key.bytes.data(), key.bytes.size()) == 1) return SIMPLER_HIP_OK;
    }

    const uint32_t q_tile = std::min<uint32_t>(num_heads, 128);  // :105
    const uint32_t q_loop = (num_heads + q_tile - 1) / q_tile;
    const uint64_t esz = 2;
    const uint32_t query_shapes[2] = {batch * num_heads, head_dim};
    const uint32_t cache_shapes[2] = {total_blocks * block_size, head_dim};
    const uint32_t out_shapes[2] = {batch * num_heads, head_dim};
    const SimplerChipTensor query = external(q.buffer.addr + q.start_offset * esz, query_shapes, 2, q.dtype);
    const SimplerChipTensor key_cache = external(kc.buffer.addr + kc.start_offset * esz, cache_shapes, 2, kc.dtype);
    const SimplerChipTensor value_cache = external(vc.buffer.addr + vc.start_offset * esz, cache_shapes, 2, vc.dtype);
    const SimplerChipTensor out =
        external(o.buffer.addr + o.start_offset * simpler_dtype_size(o.dtype), out_shapes, 2, o.dtype);
    const SimplerChipTensor block_table = bt, context_lens = cl;

    const uint32_t tile2d[2] = {q_tile, head_dim}, scalar1[1] = {q_tile}, sij2d[2] = {q_tile, block_size};
    const SimplerChipTensor tile2d_ci = create_info(tile2d, 2, SIMPLER_DT_FLOAT32);
    const SimplerChipTensor scalar_ci = create_info(scalar1, 1, SIMPLER_DT_FLOAT32);
    const SimplerChipTensor sij_ci = create_info(sij2d, 2, SIMPLER_DT_FLOAT32);
    const SimplerChipTensor pij_ci = create_info(sij2d, 2, q.dtype);

    for (uint32_t b = 0; b < batch; ++b) {
        uint64_t raw = 0;
        const uint32_t cl_idx[1] = {b};
        int rc = simpler_hip_tg_get_tensor_data(g, &context_lens, 1, cl_idx, &raw);
        if (rc != SIMPLER_HIP_OK) return rc;
        const int64_t cur_seq = (int32_t)(uint32_t)raw;
        if (cur_seq < 0 || cur_seq > (int64_t)block_num * block_size) {
            orch_log("context_lens[%u] = %lld outside [0, %llu]", b, (long long)cur_seq,
                     (unsigned long long)block_num * block_size);
            return SIMPLER_HIP_ERR_INVALID;
        }
        const uint64_t bn_this_batch = ((uint64_t)cur_seq + block_size - 1) / block_size;
        for (uint32_t qi_idx = 0; qi_idx < q_loop; ++qi_idx) {
            simpler_hip_tg_scope_begin(g);
            const uint32_t cur_offset = b * num_heads + qi_idx * q_tile;
            const uint32_t row_off[2] = {cur_offset, 0};
            const SimplerChipTensor qi = view(query, tile2d, row_off);
            const SimplerChipTensor out_view = view(out, tile2d, row_off);
            Args alloc;
            alloc.add_output(tile2d_ci);
            alloc.add_output(scalar_ci);
            alloc.add_output(scalar_ci);
            const Submitted st = submit(g, -1, alloc);  // alloc_tensors (:160-163)
            if (st.task < 0) return (int)st.task;
            const SimplerChipTensor oi = st.out[0], li_update = st.out[1], mi_update = st.out[2];
            if (bn_this_batch == 0) {
                // An empty context submits no block task, so nothing would
                // write these rows; the fused decode defines them as zeros and
                // so does this path (the reference leaves them untouched).
                Args fill;
                fill.add_output_existing(out_view);
                const Submitted zf = submit(g, FUNC_ZERO_FILL, fill);
                if (zf.task < 0) return (int)zf.task;
            }

            for (uint64_t bn = 0; bn < bn_this_batch; ++bn) {
                simpler_hip_tg_scope_begin(g);
                const uint32_t bt_idx[2] = {b, (uint32_t)bn};
                rc = simpler_hip_tg_get_tensor_data(g, &block_table, 2, bt_idx, &raw);
                if (rc != SIMPLER_HIP_OK) return rc;
                const int32_t cur_block = (int32_t)(uint32_t)raw;
                if (cur_block < 0 || (uint32_t)cur_block >= total_blocks) {
                    orch_log("block_table[%u][%llu] = %d outside the pool of %u blocks", b, (unsigned long long)bn,
                             cur_block, total_blocks);
                    return SIMPLER_HIP_ERR_BAD_BLOCK;
                }
                const uint64_t valid_len = std::min<uint64_t>(block_size, (uint64_t)cur_seq - bn * block_size);
                const uint32_t kv_shapes[2] = {block_size, head_dim};
                const uint32_t kv_offsets[2] = {(uint32_t)cur_block * block_size, 0};
                const SimplerChipTensor kj = view(key_cache, kv_shapes, kv_offsets);
                const SimplerChipTensor vj = view(value_cache, kv_shapes, kv_offsets);

                Args qk;
                qk.add_input(qi);
                qk.add_input(kj);
                qk.add_output(sij_ci);
                const Submitted qk_out = submit(g, FUNC_QK_MATMUL, qk);
                if (qk_out.task < 0) return (int)qk_out.task;
                const uint32_t valid_shapes[2] = {q_tile, (uint32_t)valid_len}, zero2[2] = {0, 0};
                const SimplerChipTensor sij_valid = view(qk_out.out[0], valid_shapes, zero2);

                Args sf;
                sf.add_input(sij_valid);
                sf.add_output(pij_ci);
                sf.add_output(scalar_ci);
                sf.add_output(scalar_ci);
                sf.add_scalar(scale_bits);
                const Submitted sf_out = submit(g, FUNC_SOFTMAX_PREPARE, sf);
                if (sf_out.task < 0) return (int)sf_out.task;

                Args pv;
                pv.add_input(sf_out.out[0]);
                pv.add_input(vj);
                pv.add_output(tile2d_ci);
                const Submitted pv_out = submit(g, FUNC_PV_MATMUL, pv);
                if (pv_out.task < 0) return (int)pv_out.task;

                Args up;
                up.add_input(sf_out.out[1]);
                up.add_input(sf_out.out[2]);
                up.add_input(pv_out.out[0]);
                up.add_inout(mi_update);
                up.add_inout(li_update);
                up.add_inout(oi);
                up.add_inout(out_view);
                up.add_scalar(bn == 0 ? 1 : 0);
                up.add_scalar(bn == bn_this_batch - 1 ? 1 : 0);
                const Submitted up_out = submit(g, FUNC_ONLINE_UPDATE, up);
                if (up_out.task < 0) return (int)up_out.task;
                simpler_hip_tg_scope_end(g);
            }
            simpler_hip_tg_scope_end(g);
        }
    }
    if (replay) return simpler_hip_tg_record_replay(g, key.bytes.data(), key.bytes.size());
    return SIMPLER_HIP_OK;
}

int simpler_hip_tg_orchestrate_vector_example(SimplerHipTaskGraph *g, const SimplerChipTensor *tensors) {
    if (!g || !tensors) return SIMPLER_HIP_ERR_INVALID;
    const SimplerChipTensor &ext_a = tensors[0], &ext_b = tensors[1], &ext_f = tensors[2];
    if (ext_a.ndims < 1) return SIMPLER_HIP_ERR_INVALID;
    simpler_hip_tg_bind(g, 0, SIMPLER_HIP_K_VEC_ADD);
    simpler_hip_tg_bind(g, 1, SIMPLER_HIP_K_VEC_ADD_SCALAR);
    simpler_hip_tg_bind(g, 2, SIMPLER_HIP_K_VEC_MUL);
    // GRAPH mode: the step depends on its three tensors only
    StepKey key;
    const bool replay = replayable(g);
    if (replay) {
        key.add(tensors, 3 * sizeof(SimplerChipTensor));
        if (simpler_hip_tg_replay(g, key.bytes.data(), key.bytes.size()) == 1) return SIMPLER_HIP_OK;
    }
    const uint32_t size = ext_a.shapes[0];
    const SimplerChipTensor inter_ci = create_info(&size, 1, SIMPLER_DT_FLOAT32);

    Args t0;  // c = a + b
    t0.add_input(ext_a);
    t0.add_input(ext_b);
    t0.add_output(inter_ci);
    const Submitted o0 = submit(g, 0, t0);
    if (o0.task < 0) return (int)o0.task;
    const SimplerChipTensor c = o0.out[0];

    simpler_hip_tg_scope_begin(g);
    Args t1;  // d = c + 1
    t1.add_input(c);
    t1.add_output(inter_ci);
    t1.add_scalar(f32_bits(1.0f));
    t1.add_scalar(3u);
    const Submitted o1 = submit(g, 1, t1);
    if (o1.task < 0) return (int)o1.task;
    Args t2;  // e = c + 2
    t2.add_input(c);
    t2.add_output(inter_ci);
    t2.add_scalar(f32_bits(2.0f));
    t2.add_scalar(3u);
    const Submitted o2 = submit(g, 1, t2);
    if (o2.task < 0) return (int)o2.task;
    Args t3;  // g = d * e
    t3.add_input(o1.out[0]);
    t3.add_input(o2.out[0]);
    t3.add_output(inter_ci);
    t3.add_scalar(3u);
    const Submitted o3 = submit(g, 2, t3);
    if (o3.task < 0) return (int)o3.task;
    Args t4;  // f = g + c
    t4.add_input(o3.out[0]);
    t4.add_input(c);
    t4.add_output_existing(ext_f);
    const Submitted o4 = submit(g, 0, t4);
    if (o4.task < 0) return (int)o4.task;
    simpler_hip_tg_scope_end(g);
    if (replay) return simpler_hip_tg_record_replay(g, key.bytes.data(), key.bytes.size());
    return SIMPLER_HIP_OK;
}

}  // extern "C"
