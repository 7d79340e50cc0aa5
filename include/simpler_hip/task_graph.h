/* Task-graph backend: simpler's tensormap-and-ringbuffer task model on one
 * HIP device (gfx950 / MI355X).
 *
 * An orchestration submits tasks one by one. Each task names an incore kernel
 * and carries tagged ChipTensor arguments and u64 scalars, in the order the
 * kernel reads them, exactly as simpler's CoreTaskArgs does
 * (src/a2a3/runtime/tensormap_and_ringbuffer/runtime/pto_types.h:374-398,507;
 * tags from src/common/task_interface/tensor.h:43-49). Dependencies are
 * inferred the way simpler's submit_task does
 * (runtime/pto_orchestrator.cpp:882-1254, runtime/pto_dep_compute.h):
 *   - a non-OUTPUT tensor whose owner_task_id names a task of this graph
 *     depends on that task (creator edge);
 *   - INPUT and INOUT tensors (manual_dep clear) depend on every earlier
 *     INOUT / OUTPUT_EXISTING writer of an overlapping view of the same buffer
 *     (TensorMap lookup, runtime/pto_tensormap.h check_overlap: same
 *     buffer.addr; views of one row-major layout compared per dimension,
 *     others by byte range [offset, offset + extent)); an INOUT that contains
 *     an older writer's view retires that entry;
 *   - INOUT and OUTPUT_EXISTING tensors (manual_dep clear) are published as
 *     the newest writer of their range;
 *   - OUTPUT tensors are allocated by the runtime (row-major, device memory)
 *     and owned by the submitting task;
 *   - explicit dependencies (Arg::set_dependencies) are added as given.
 * Runtime-allocated tensors live until the end of the innermost scope open at
 * allocation (PTO2_SCOPE, pto_orchestration_api.h:335-369); a later
 * allocation that reuses their memory depends on every task that touched it.
 *
 * Modes:
 *   EAGER        each task is launched on the graph's stream as it is
 *                submitted (stream order is a topological order of the DAG);
 *   GRAPH        tasks become nodes of a hipGraph whose edges are the inferred
 *                dependencies; simpler_hip_tg_launch instantiates (or updates)
 *                and launches it. Reading tensor data that a pending task
 *                produces first launches and drains the graph built so far.
 *   RECORD_ONLY  no device work at all: dependencies and allocations are
 *                computed (addresses are placeholders) for inspection.
 *
 * All functions return 0 / a non-negative id, or a negative SIMPLER_HIP_ERR_*
 * code (the reason is printed to stderr). A graph is used from one thread.
 */
#ifndef SIMPLER_HIP_TASK_GRAPH_H
#define SIMPLER_HIP_TASK_GRAPH_H

#include <stdint.h>

#include "simpler_hip/abi_types.h"
#include "simpler_hip/pa_decode.h" /* error codes */

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

/* TensorArgType (src/common/task_interface/tensor.h:43-49). */
typedef enum SimplerHipTensorArgType {
    SIMPLER_HIP_TA_INPUT = 0,
    SIMPLER_HIP_TA_OUTPUT = 1,
    SIMPLER_HIP_TA_INOUT = 2,
    SIMPLER_HIP_TA_OUTPUT_EXISTING = 3,
    SIMPLER_HIP_TA_NO_DEP = 4
} SimplerHipTensorArgType;

/* Built-in incore kernels. Tensor arguments in order, then scalars:
 *   QK_MATMUL       qi [M,K] bf16, kj [N,K] bf16, sij [M,N] f32 (out)
 *                   <- examples/a2a3/tensormap_and_ringbuffer/paged_attention/kernels/aic/aic_qk_matmul.cpp:38-115
 *   SOFTMAX_PREPARE sij [M,valid] f32 view, pij [M,N] bf16 (out), mij [M] f32 (out), lij [M] f32 (out);
 *                   scalar scale (f32 bits)
 *                   <- .../aiv/aiv_softmax_prepare.cpp:45-156
 *   PV_MATMUL       pij [M,N] bf16, vj [N,D] bf16, oi_new [M,D] f32 (out)
 *                   <- .../aic/aic_pv_matmul.cpp:38-114
 *   ONLINE_UPDATE   mij, lij [M] f32, oi_new [M,D] f32, mi, li [M] f32 (inout), oi [M,D] f32 (inout),
 *                   dst [M,D] f32 or bf16 (inout); scalars is_first, is_last
 *                   <- .../aiv/aiv_online_update.cpp:40-256
 *   VEC_ADD         a, b, c (out), f32, same element count: c = a + b
 *                   <- examples/a2a3/tensormap_and_ringbuffer/vector_example/kernels/aiv/kernel_add.cpp
 *   VEC_ADD_SCALAR  a, c (out), f32; scalar s (f32 bits): c = a + s
 *                   <- .../vector_example/kernels/aiv/kernel_add_scalar.cpp
 *   VEC_MUL         a, b, c (out), f32: c = a * b
 *                   <- .../vector_example/kernels/aiv/kernel_mul.cpp
 *   ZERO_FILL       dst [M,D] f32 or bf16 (out): dst = 0. No reference counterpart: the
 *                   paged-attention orchestration writes it for an empty context, whose
 *                   output the fused decode defines as zeros.
 * Matrix operands need unit stride in their last dimension. */
typedef enum SimplerHipIncoreKernel {
    SIMPLER_HIP_K_QK_MATMUL = 0,
    SIMPLER_HIP_K_SOFTMAX_PREPARE = 1,
    SIMPLER_HIP_K_PV_MATMUL = 2,
    SIMPLER_HIP_K_ONLINE_UPDATE = 3,
    SIMPLER_HIP_K_VEC_ADD = 16,
    SIMPLER_HIP_K_VEC_ADD_SCALAR = 17,
    SIMPLER_HIP_K_VEC_MUL = 18,
    SIMPLER_HIP_K_ZERO_FILL = 19
} SimplerHipIncoreKernel;

typedef enum SimplerHipTaskGraphMode {
    SIMPLER_HIP_TG_EAGER = 0,
    SIMPLER_HIP_TG_GRAPH = 1,
    SIMPLER_HIP_TG_RECORD_ONLY = 2
} SimplerHipTaskGraphMode;

/* PTO2TaskId::invalid() (src/common/task_interface/pto_task_id.h:31-40):
 * owner_task_id of external tensors. Tasks of a graph get ids 0, 1, 2, ...
 * (ring 0, local id = submission index). */
#define SIMPLER_HIP_TASK_INVALID UINT64_MAX

typedef struct SimplerHipTaskGraph SimplerHipTaskGraph;

/* A graph on the current HIP device; `stream` (hipStream_t, NULL = default)
 * carries all of its work. RECORD_ONLY needs no device. NULL on failure. */
SimplerHipTaskGraph *simpler_hip_tg_create(int32_t mode, void *stream);
/* Waits for outstanding work, then frees the graph and its device memory. */
void simpler_hip_tg_destroy(SimplerHipTaskGraph *g);

/* Map func_id (0..63, the id an orchestration submits, e.g. FUNC_QK_MATMUL)
 * to a built-in kernel. Unbound ids are rejected at submit. */
int simpler_hip_tg_bind(SimplerHipTaskGraph *g, int32_t func_id, int32_t kernel);

/* ---- Kernels of the caller's own ----
 * A registered kernel is a gfx950 `extern "C" __global__` function in a code
 * object file (hipcc --genco), taking one by-value SimplerHipKernelArgs: the
 * task's tensors in submission order as the kernel sees them (OUTPUT tensors
 * materialised by the runtime), then its scalars. This is the reference's
 * incore entry convention, `kernel_entry(int64_t *args)` with the task's
 * ChipTensors first and its scalars after them
 * (examples/a2a3/tensormap_and_ringbuffer/vector_example/kernels/aiv/kernel_add.cpp:49-55),
 * as one HIP kernel argument instead of a pointer to a device-side array. */
#define SIMPLER_HIP_TG_KERNEL_MAX_TENSORS SIMPLER_CORE_MAX_TENSOR_ARGS

typedef struct SimplerHipKernelTensor {
    uint64_t addr;   /* device address of the view's first element (buffer.addr + start_offset * element size) */
    uint32_t ndims;
    uint32_t dtype;  /* SimplerDataType */
    uint32_t shapes[SIMPLER_MAX_TENSOR_DIMS];
    uint32_t strides[SIMPLER_MAX_TENSOR_DIMS]; /* elements */
} SimplerHipKernelTensor;

typedef struct SimplerHipKernelArgs {
    int32_t n_tensors;
    int32_t n_scalars;
    SimplerHipKernelTensor tensors[SIMPLER_HIP_TG_KERNEL_MAX_TENSORS];
    uint64_t scalars[SIMPLER_CORE_MAX_SCALAR_ARGS];
} SimplerHipKernelArgs;

/* Bind func_id to kernel `kernel_name` of the code object at
 * `code_object_path` (loaded once per path and graph, on the graph's device).
 * Replaces the reference's per-callable child binaries resolved at
 * registration (src/common/task_interface/callable.h:99-163) and dispatched
 * by func id from rt_submit_task (orchestration/pto_orchestration_api.h:170-194).
 * Launch shape of each task: `block_threads` threads per workgroup (1..1024);
 * grid = ceil(numel(tensor `grid_tensor`) / elems_per_workgroup) workgroups
 * (at least 1), or exactly elems_per_workgroup workgroups when grid_tensor < 0.
 * Tasks may pass any tensors of device memory (at most
 * SIMPLER_HIP_TG_KERNEL_MAX_TENSORS) and scalars; checking their shapes is the
 * kernel's business. Returns SIMPLER_HIP_ERR_INVALID for a bad argument and
 * SIMPLER_HIP_ERR_UNSUPPORTED when the file or kernel cannot be loaded. */
int simpler_hip_tg_register_kernel(SimplerHipTaskGraph *g, int32_t func_id, const char *code_object_path,
                                   const char *kernel_name, uint32_t block_threads, int32_t grid_tensor,
                                   uint32_t elems_per_workgroup);

int simpler_hip_tg_scope_begin(SimplerHipTaskGraph *g);
int simpler_hip_tg_scope_end(SimplerHipTaskGraph *g);

/* Submit one task (rt_submit_task, pto_orchestration_api.h:170-209).
 * tensors[i] with arg_types[i] == OUTPUT is a create info: only ndims,
 * shapes and dtype are read. outputs (n_tensors entries, may be NULL)
 * receives every argument as the kernel sees it, with OUTPUT slots
 * materialised (device address, owner_task_id = the new task).
 * func_id < 0 submits a dependency-only task (rt_submit_dummy_task).
 * Returns the task id. */
int64_t simpler_hip_tg_submit(SimplerHipTaskGraph *g, int32_t func_id, const SimplerChipTensor *tensors,
                              const int32_t *arg_types, int32_t n_tensors, const uint64_t *scalars,
                              int32_t n_scalars, const uint64_t *explicit_deps, int32_t n_explicit_deps,
                              SimplerChipTensor *outputs);

/* Allocate tensors without a kernel (alloc_tensors, pto_orchestration_api.h:120-168):
 * a dependency-only task owns them. Returns its id. */
int64_t simpler_hip_tg_alloc(SimplerHipTaskGraph *g, const SimplerChipTensor *create_infos, int32_t n,
                             SimplerChipTensor *outputs);

/* Element of a tensor as raw bits (get_tensor_data, pto_orchestration_api.h:269-291):
 * waits for the tensor's producers first. *value receives the element's
 * bytes zero-extended to 64 bits. */
int simpler_hip_tg_get_tensor_data(SimplerHipTaskGraph *g, const SimplerChipTensor *t, uint32_t ndims,
                                   const uint32_t *indices, uint64_t *value);

/* Copy a tensor's bytes [start_offset, start_offset + extent) (elements
 * times the dtype size) to host memory, after its producers have finished.
 * `bytes` must cover that range. */
int simpler_hip_tg_copy_to_host(SimplerHipTaskGraph *g, const SimplerChipTensor *t, void *host, uint64_t bytes);

/* GRAPH mode: instantiate (or update) and launch the pending graph. EAGER and
 * RECORD_ONLY: nothing to do. Asynchronous on the graph's stream. */
int simpler_hip_tg_launch(SimplerHipTaskGraph *g);
/* Wait until everything launched so far has finished. */
int simpler_hip_tg_wait(SimplerHipTaskGraph *g);
/* Forget all tasks and recycle all runtime-allocated memory (waits first).
 * Bindings and the instantiated graph (for update on the next launch) stay. */
int simpler_hip_tg_reset(SimplerHipTaskGraph *g);

/* ---- Whole-step replay (GRAPH mode) ----
 * A step orchestrated from a reset graph is a function of what its
 * orchestration reads: the tensors it is given, its scalars, and the values it
 * reads with get_tensor_data. The caller names those in `key`.
 *   record_replay  after the step's tasks are submitted and before its launch:
 *                  keep the graph's state under `key` (one key per graph; a
 *                  new record replaces the old one). The step must have started
 *                  on a reset (or new) graph, possibly inside open scopes that
 *                  held nothing yet, and nothing may have been launched since;
 *                  `key` must determine every task submitted since the reset.
 *   replay         on a reset graph (the same depth of open, empty scopes as
 *                  at the recorded step's start): if `key` equals the recorded
 *                  one, restore that state (tasks, dependencies, allocations,
 *                  scopes) and return 1; simpler_hip_tg_launch then runs the
 *                  cached executable graph without any task being submitted
 *                  again. Otherwise return 0 and change nothing.
 * No counterpart in the reference, whose orchestration runs on the device
 * each step; here it runs on the host, and a decode loop re-submits the same
 * DAG every step. EAGER and RECORD_ONLY graphs never replay (replay returns 0,
 * record_replay does nothing). */
int simpler_hip_tg_record_replay(SimplerHipTaskGraph *g, const void *key, uint64_t key_bytes);
int simpler_hip_tg_replay(SimplerHipTaskGraph *g, const void *key, uint64_t key_bytes);

/* Orchestrations of the reference's examples, run against graph `g` (which
 * gets its func ids bound). Tensors are in the callable's order; kernel
 * operands must be device memory, tables read only through get_tensor_data
 * may be host memory.
 *   paged attention  <- examples/a2a3/tensormap_and_ringbuffer/paged_attention/kernels/orchestration/
 *                       paged_attention_orch.cpp:77-249: query [B,Hq,D] bf16, key_cache / value_cache
 *                       [nblk,BS,D] or [nblk,BS,1,D] bf16, block_table [B,maxblk] i32,
 *                       context_lens [B] i32, out [B,Hq,D] f32 or bf16; scale as f32 bits.
 *                       Per (sequence, 128-head tile) and KV block: QK -> SF -> PV -> UP.
 *   vector example   <- examples/a2a3/tensormap_and_ringbuffer/vector_example/kernels/orchestration/
 *                       example_orchestration.cpp:55-112: a, b, f fp32 [n]; f = (a+b+1)*(a+b+2) + (a+b).
 * In GRAPH mode on a reset graph, both record their step for replay, keyed on
 * the tensors, the scale and (paged attention) every context_lens and
 * block_table value they read: a repeated step with the same tables replays
 * its cached graph without being orchestrated again. */
int simpler_hip_tg_orchestrate_paged_attention(SimplerHipTaskGraph *g, const SimplerChipTensor *tensors,
                                               uint64_t scale_bits);
int simpler_hip_tg_orchestrate_vector_example(SimplerHipTaskGraph *g, const SimplerChipTensor *tensors);

/* Inspection: number of tasks; the steps replayed so far; the producers task
 * `task` waits on (sorted, at most cap written; returns the full count); bytes
 * of device memory the graph holds for runtime-allocated tensors. */
int64_t simpler_hip_tg_task_count(const SimplerHipTaskGraph *g);
/* Steps restored by simpler_hip_tg_replay over the graph's lifetime. */
uint64_t simpler_hip_tg_replay_count(const SimplerHipTaskGraph *g);
int32_t simpler_hip_tg_fanin(const SimplerHipTaskGraph *g, int64_t task, int64_t *producers, int32_t cap);
uint64_t simpler_hip_tg_arena_bytes(const SimplerHipTaskGraph *g);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* SIMPLER_HIP_TASK_GRAPH_H */
