/*
 * simpler_hip — the host-runtime C API exported by libsimpler_hip.so.
 *
 * Same symbol names, signatures and return conventions as the reference's
 * canonical host-runtime header, so simpler's ChipWorker can dlopen this
 * library in place of an Ascend/sim host_runtime.so and resolve every symbol it
 * requires (reference: src/common/worker/pto_runtime_c_api.h:188-478; the
 * dlsym list is src/common/worker/chip_worker.cpp:205-256).
 *
 * Backend specifics:
 *  - One HIP device and one HIP stream per device context.
 *  - simpler_register_callable accepts the paged-attention ChipCallable (the
 *    QK/SF/PV/UP chain of examples/a2a3/tensormap_and_ringbuffer/
 *    paged_attention/test_paged_attention.py:25-61, or a callable named
 *    "simpler_hip_paged_attention_decode") and runs it as one fused kernel;
 *    other callables return PTO_RUNTIME_ERR_UNSUPPORTED.
 *  - aicpu/aicore/dispatcher binaries passed to simpler_init are ignored.
 *  - Communication, ACL and DMA-workspace entry points are not part of this
 *    single-GPU backend and return PTO_RUNTIME_ERR_UNSUPPORTED (or NULL / 0).
 *
 * Error codes: 0 = success, negative = error.
 */
#ifndef SIMPLER_HIP_PTO_RUNTIME_C_API_H
#define SIMPLER_HIP_PTO_RUNTIME_C_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

typedef void *RuntimeHandle;
typedef void *DeviceContextHandle;
typedef struct CommHandle_ *CommHandle;
typedef struct CommGlobalDomainDescriptor CommGlobalDomainDescriptor;
struct CallConfig; /* byte layout: SimplerCallConfig in abi_types.h */

enum {
    PTO_RUNTIME_ERR_UNSUPPORTED = -2,
    PTO_RUNTIME_ERR_PREPARED_INCOMPATIBLE = -3,
};

enum {
    SIMPLER_NATIVE_RUN_POLL_ERROR = -1,
    SIMPLER_NATIVE_RUN_POLL_NOT_READY = 0,
    SIMPLER_NATIVE_RUN_POLL_COMPLETE = 1,
};

enum {
    PTO_PIPELINE_CONTRACT_ABI_VERSION = 1,
    PTO_PIPELINE_MAX_RESOURCES = 8,
    PTO_PIPELINE_MAX_DEPTH = 2,
};

typedef struct PipelineResource {
    uint32_t kind;
    uint32_t resource_class;
    uint64_t bytes_per_copy;
} PipelineResource;

typedef struct PipelineContract {
    uint32_t abi_version;
    uint32_t resource_count;
    uint32_t pipeline_depth;
    PipelineResource resources[PTO_PIPELINE_MAX_RESOURCES];
} PipelineContract;

typedef struct NativeRunDescriptor {
    uint32_t pipeline_slot;
    uint32_t arena_bank;
    uint64_t run_id;
    uint64_t generation;
    uint64_t dispatch_id;
    uint64_t run_epoch;
    volatile int32_t *accepted_state;
    int32_t accepted_value;
} NativeRunDescriptor;

/* pipeline / sizing (pto_runtime_c_api.h:188-225) */
const PipelineContract *get_pipeline_contract(void);
size_t get_runtime_size(void);
size_t get_runtime_alignment(void);

/* lifecycle (:193-199, :264-272) */
DeviceContextHandle create_device_context(void);
void destroy_device_context(DeviceContextHandle ctx);
int simpler_init(DeviceContextHandle ctx, int device_id, const uint8_t *aicpu_binary, size_t aicpu_size,
                 const uint8_t *aicore_binary, size_t aicore_size, const uint8_t *dispatcher_binary,
                 size_t dispatcher_size, const struct CallConfig *prewarm_config);
int finalize_device(DeviceContextHandle ctx);

/* device memory (:228-252) */
void *device_malloc_ctx(DeviceContextHandle ctx, size_t size);
void device_free_ctx(DeviceContextHandle ctx, void *dev_ptr);
size_t committed_device_memory_ctx(DeviceContextHandle ctx);
int copy_to_device_ctx(DeviceContextHandle ctx, void *dev_ptr, const void *host_ptr, size_t size);
int copy_from_device_ctx(DeviceContextHandle ctx, void *host_ptr, const void *dev_ptr, size_t size);

/* callables and runs (:285-420) */
int simpler_register_callable(DeviceContextHandle ctx, int32_t callable_id, const void *callable);
int simpler_unregister_callable(DeviceContextHandle ctx, int32_t callable_id);
int simpler_run(DeviceContextHandle ctx, RuntimeHandle runtime, int32_t callable_id, const void *args,
                const struct CallConfig *config, const NativeRunDescriptor *descriptor);
int simpler_prepare_run(DeviceContextHandle ctx, RuntimeHandle runtime, int32_t callable_id, const void *args,
                        const struct CallConfig *config, const NativeRunDescriptor *descriptor);
int supports_concurrent_native_prepare_ctx(DeviceContextHandle ctx);
int simpler_launch_run(DeviceContextHandle ctx, RuntimeHandle runtime);
int simpler_poll_run(DeviceContextHandle ctx, RuntimeHandle runtime);
int simpler_wait_run(DeviceContextHandle ctx, RuntimeHandle runtime);
int simpler_finalize_run(DeviceContextHandle ctx, RuntimeHandle runtime);
uint64_t get_arena_bank_gm_heap_base_ctx(DeviceContextHandle ctx, uint32_t bank_id);
uint64_t get_retained_temp_addr_ctx(DeviceContextHandle ctx, uint32_t slot_id);
size_t get_aicpu_dlopen_count(DeviceContextHandle ctx);
size_t get_host_dlopen_count(DeviceContextHandle ctx);
size_t get_run_stream_set_create_count(DeviceContextHandle ctx);
int simpler_provision_dma_workspace(DeviceContextHandle ctx, uint32_t required_mask, const void *sdma_warmup_binary,
                                    uint64_t sdma_warmup_size);

/* ACL / comm streams (src/a2a3/platform/sim/host/pto_runtime_c_api.cpp:41-55) */
int ensure_acl_ready_ctx(DeviceContextHandle ctx, int device_id);
void *create_comm_stream_ctx(DeviceContextHandle ctx);
int destroy_comm_stream_ctx(DeviceContextHandle ctx, void *stream);

/* comm (src/common/platform_comm/comm.h:144-332) — unsupported on this backend */
CommHandle comm_init(int rank, int nranks, void *stream, const char *rootinfo_path);
int comm_alloc_windows(CommHandle h, size_t win_size, uint64_t *device_ctx_out);
int comm_get_local_window_base(CommHandle h, uint64_t *base_out);
int comm_get_window_size(CommHandle h, size_t *size_out);
int comm_derive_context(CommHandle h, const uint32_t *rank_ids, size_t rank_count, uint32_t domain_rank,
                        size_t window_offset, size_t window_size, uint64_t *device_ctx_out);
int comm_alloc_domain_windows(CommHandle h, uint64_t allocation_id, const uint32_t *rank_ids, size_t rank_count,
                              uint32_t domain_rank, size_t window_size, uint64_t *device_ctx_out,
                              uint64_t *local_window_base_out);
int comm_release_domain_windows(CommHandle h, uint64_t allocation_id, size_t rank_count, uint32_t domain_rank);
int comm_global_domain_prepare(uint64_t domain_id, uint32_t domain_rank, uint32_t rank_count, size_t window_size,
                               uint32_t profile, CommGlobalDomainDescriptor *descriptor_out,
                               uint64_t *local_window_base_out);
int comm_global_domain_import(uint64_t domain_id, const CommGlobalDomainDescriptor *descriptors,
                              size_t descriptor_count, uint64_t *device_ctx_out);
int comm_global_domain_release(uint64_t domain_id);
int comm_barrier(CommHandle h);
int comm_destroy(CommHandle h);

/* simpler_hip extension (no reference counterpart): the HIP stream of a
 * context, so callers can order their own work against simpler_run. */
void *simpler_hip_context_stream(DeviceContextHandle ctx);

/* simpler_hip extension (no reference counterpart): how a context executes a
 * paged-attention callable from now on. FUSED (default): the fused split-K
 * decode kernel. TASK_GRAPH: the reference's orchestration (QK -> SF -> PV ->
 * UP per KV block) on the task-graph backend, each task launched as it is
 * submitted. TASK_GRAPH_HIPGRAPH: the same DAG captured as one hipGraph with
 * the inferred dependencies as edges. SIMPLER_HIP_EXECUTION=eager|graph in the
 * environment at simpler_init selects the same. Returns 0 or -1. */
enum { SIMPLER_HIP_EXEC_FUSED = 0, SIMPLER_HIP_EXEC_TASK_GRAPH = 1, SIMPLER_HIP_EXEC_TASK_GRAPH_HIPGRAPH = 2 };
int simpler_hip_set_execution(DeviceContextHandle ctx, int32_t execution);

/* simpler_hip extension (no reference counterpart): which paged-attention
 * callable family registration id `callable_id` matched, or -1 (not
 * registered, or not paged attention). CHAIN: the per-block QK/SF/PV/UP
 * chain (examples/a2a3/tensormap_and_ringbuffer/paged_attention and its
 * manual_scope / ringbuffer / batch / multi_round variants); UNROLL: the
 * grouped split-K chain whose QK and PV take three inputs (paged_attention_unroll,
 * *_unroll_manual_scope, *_unroll_4dims); SPMD: the cooperative AIC/AIV task
 * (spmd_paged_attention); NATIVE: the callable named
 * simpler_hip_paged_attention_decode; HIGHPERF: the high-performance SPMD
 * task (spmd_paged_attention_highperf: query, caches, block_table, out,
 * workspaces, a tiling tensor carrying the lengths and the scale). All run on
 * the fused decode kernel. */
enum {
    SIMPLER_HIP_PA_CHAIN = 0,
    SIMPLER_HIP_PA_UNROLL = 1,
    SIMPLER_HIP_PA_SPMD = 2,
    SIMPLER_HIP_PA_NATIVE = 3,
    SIMPLER_HIP_PA_HIGHPERF = 4
};
int simpler_hip_callable_family(DeviceContextHandle ctx, int32_t callable_id);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* SIMPLER_HIP_PTO_RUNTIME_C_API_H */
