// Task-graph backend runtime: dependency inference, scoped device memory and
// execution of incore-kernel tasks on one HIP device.
//
// Dependency rules follow simpler's submit path
// (src/a2a3/runtime/tensormap_and_ringbuffer/runtime/pto_orchestrator.cpp:882-1254):
//   explicit deps            (:959-984)
//   creator edge + TensorMap lookup for INPUT/INOUT, INOUT covering an older
//   writer retires it        (runtime/pto_dep_compute.h compute_task_fanin)
//   INOUT / OUTPUT_EXISTING published as the newest writer
//                            (pto_dep_compute.h register_task_outputs)
// The TensorMap here is a hash map from buffer address to the writer regions
// on that buffer. Overlap follows runtime/pto_tensormap.h check_overlap: views
// of one canonical layout are compared as per-dimension boxes, anything else
// by byte range [offset, offset + extent) (conservative: it may add an edge,
// never drop one). The reference's ring-buffer entry pool and lazy
// invalidation exist because the AICPU cannot allocate; here the host can.
//
// Memory: runtime-allocated OUTPUT tensors come from grow-only device chunks.
// Closing a scope returns the scope's tensors to a free list together with
// every task that touched them; whoever reuses that memory depends on those
// tasks (the write-after-read order simpler gets from its ring buffers'
// fanout reference counts, pto_ring_buffer.h).
//
// Execution: EAGER launches each task on the stream at submit. GRAPH turns the
// tasks submitted between launches (a segment) into one hipGraph, a kernel
// node per task. The nodes form one chain in submission order (a topological
// order of the inferred DAG), the order EAGER runs them in: on cfg1 a graph
// with the DAG's own edges cost 146 µs of host time per hipGraphLaunch and
// 212 µs on the device, the chain 55 and 147 µs (ROCm runs a DAG's branches
// on internal streams joined by waits). The inferred edges still decide when
// a cached graph may be replayed. The executable
// graph is cached per segment index: when the next run submits the same
// kernels, launch shapes and edges (a decode loop over stable buffers), it is
// replayed, with hipGraphExecKernelNodeSetParams on the nodes whose parameter
// blocks changed, instead of being rebuilt. A whole step can also be replayed
// without being submitted again: record_replay keeps the graph's state after a
// step's orchestration under a caller key, and replay restores it on a reset
// graph, so only the launch of the cached executable graph is left.
//
// Kernels: the built-in incore kernels (incore_kernels.hip), plus kernels the
// caller registers from code object files; those get the task's tensors and
// scalars as one SimplerHipKernelArgs.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <deque>
#include <map>
#include <new>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <string>
#include <unordered_map>
#include <vector>

#include "incore.h"
#include "simpler_hip/task_graph.h"
#include "task_graph_internal.h"

namespace {

using simpler_hip::KernelLaunch;

constexpr int kMaxFuncIds = 64;
constexpr int32_t kCustomBase = 1 << 20;  // kernel codes of registered kernels: kCustomBase + index
constexpr size_t kAlign = 256;
constexpr size_t kChunkBytes = (size_t)64 << 20;
constexpr uint64_t kRecordBase = 0x7e0000000000ull;  // placeholder device addresses in RECORD_ONLY mode

void tg_log(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "[simpler_hip task_graph] ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
}

struct Task {
    int32_t func_id = -1;
    int32_t kernel = -1;  // -1: dependency-only
    KernelLaunch launch;  // launch.func: a __global__ stub, or the hipFunction_t of a registered kernel
    std::vector<int32_t> fanin;
};

// A kernel registered from a code object: its function and launch shape rule.
struct CustomKernel {
    hipFunction_t fn = nullptr;
    uint32_t block = 64;
    int32_t grid_tensor = -1;
    uint32_t per_wg = 1;
};

// One node of a cached executable graph: what must match for a replay.
struct NodeSig {
    const void *func = nullptr;
    size_t param_bytes = 0;
    unsigned grid = 0, block = 0;
    std::vector<int32_t> deps;  // producers, as indices within the segment
};

struct SegmentCache {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<hipGraphNode_t> nodes;
    std::vector<NodeSig> sigs;
    std::vector<std::vector<unsigned char>> params;  // each node's parameter block as last set
    void clear() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
        nodes.clear();
        sigs.clear();
        params.clear();
    }
};

// A writer's view of a buffer: its byte range plus the geometry needed for
// the per-dimension test.
struct Region {
    uint64_t begin, end;  // bytes from the buffer address
    uint64_t start;       // elements
    uint32_t esz, ndims;
    uint32_t shapes[SIMPLER_MAX_TENSOR_DIMS];
    uint32_t strides[SIMPLER_MAX_TENSOR_DIMS];
    int32_t producer;
};

struct Buffer {
    uint64_t addr;
    size_t bytes;
    std::vector<int32_t> users;  // owner first, then every task that named the tensor
};

struct FreeBlock {
    uint64_t addr;
    size_t bytes;
    std::vector<int32_t> retire;
};

struct Chunk {
    void *base;
    size_t bytes;
    size_t used;
};

// A host copy of an external tensor's bytes [begin, end), in pinned memory
// (one asynchronous copy and one stream synchronisation per refresh).
struct HostCopy {
    uint64_t begin = 0, end = 0;  // bytes from the buffer address
    uint8_t *data = nullptr;      // hipHostMalloc'ed, `cap` bytes
    size_t cap = 0;
    bool valid = false;
};

// The state of a graph after one step's orchestration, kept for replay.
struct StepSnapshot {
    bool valid = false;
    std::vector<uint8_t> key;
    std::deque<Task> tasks;
    std::unordered_map<uint64_t, std::vector<Region>> tmap;
    std::unordered_map<uint64_t, int32_t> buf_of;
    std::vector<Buffer> bufs;
    std::vector<std::vector<int32_t>> scopes;
    std::multimap<size_t, FreeBlock> free_blocks;
    std::vector<size_t> chunk_used;
    size_t chunk_cursor = 0;
    uint64_t record_next = 0;
};

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

bool valid_tensor(const SimplerChipTensor &t) {
    if (t.ndims == 0 || t.ndims > SIMPLER_MAX_TENSOR_DIMS || simpler_dtype_size(t.dtype) == 0) return false;
    for (uint32_t d = 0; d < t.ndims; ++d)
        if (t.strides[d] == 0 && t.shapes[d] > 1) return false;
    return true;
}

void byte_range(const SimplerChipTensor &t, uint64_t *b, uint64_t *e) {
    const uint64_t esz = simpler_dtype_size(t.dtype);
    *b = t.start_offset * esz;
    *e = *b + extent_elems(t) * esz;
}

bool dense(const SimplerChipTensor &t) {
    uint64_t expect = 1;
    for (int d = (int)t.ndims - 1; d >= 0; --d) {
        if (t.shapes[d] != 1 && t.strides[d] != expect) return false;
        expect *= t.shapes[d];
    }
    return true;
}

Region region_of(const SimplerChipTensor &t, int32_t producer) {
    Region r;
    memset(&r, 0, sizeof(r));
    byte_range(t, &r.begin, &r.end);
    r.start = t.start_offset;
    r.esz = (uint32_t)simpler_dtype_size(t.dtype);
    r.ndims = t.ndims;
    for (uint32_t d = 0; d < t.ndims; ++d) {
        r.shapes[d] = t.shapes[d];
        r.strides[d] = t.strides[d];
    }
    r.producer = producer;
    return r;
}

enum class Overlap { kNone, kCovered, kOther };

// Per-dimension offsets of a view on a canonical layout (strides descending,
// each a multiple of the next): the view is the box [off_d, off_d + shape_d)
// when no dimension wraps into the next.
bool box_of(uint64_t start, uint32_t nd, const uint32_t *shapes, const uint32_t *strides, uint64_t *off) {
    for (uint32_t d = 0; d < nd; ++d) {
        if (strides[d] == 0) return false;
        if (d > 0 && strides[d - 1] % strides[d] != 0) return false;
    }
    for (uint32_t d = 0; d < nd; ++d) {
        uint64_t q = start / strides[d];
        if (d > 0) {
            const uint64_t extent = strides[d - 1] / strides[d];
            q %= extent;
            if (q + shapes[d] > extent) return false;
        }
        off[d] = q;
    }
    return true;
}

// How a reader/writer view `in` relates to a writer region `r` on the same
// buffer (runtime/pto_tensormap.h check_overlap: kCovered = `in` contains `r`).
// Views with the same canonical geometry are compared box by box; anything
// else by byte range, where only a dense `in` can cover.
Overlap overlap(const Region &r, const SimplerChipTensor &in) {
    uint64_t b, e;
    byte_range(in, &b, &e);
    if (!(r.end > b && e > r.begin)) return Overlap::kNone;
    bool same = r.esz == simpler_dtype_size(in.dtype) && r.ndims == in.ndims;
    for (uint32_t d = 0; same && d < r.ndims; ++d) same = r.strides[d] == in.strides[d];
    uint64_t ro[SIMPLER_MAX_TENSOR_DIMS], io[SIMPLER_MAX_TENSOR_DIMS];
    if (same && box_of(r.start, r.ndims, r.shapes, r.strides, ro) &&
        box_of(in.start_offset, in.ndims, in.shapes, in.strides, io)) {
        bool contains = true;
        for (uint32_t d = 0; d < r.ndims; ++d) {
            const uint64_t re = ro[d] + r.shapes[d], ie = io[d] + in.shapes[d];
            if (!(re > io[d] && ie > ro[d])) return Overlap::kNone;
            if (!(io[d] <= ro[d] && re <= ie)) contains = false;
        }
        return contains ? Overlap::kCovered : Overlap::kOther;
    }
    return (dense(in) && b <= r.begin && r.end <= e) ? Overlap::kCovered : Overlap::kOther;
}

}  // namespace

struct SimplerHipTaskGraph {
    int32_t mode = SIMPLER_HIP_TG_EAGER;
    hipStream_t stream = nullptr;
    int device = -1;
    int32_t func_kernel[kMaxFuncIds];
    std::deque<Task> tasks;  // stable addresses: graph nodes keep pointing at their parameter blocks
    std::unordered_map<uint64_t, std::vector<Region>> tmap;
    std::unordered_map<uint64_t, int32_t> buf_of;  // address -> index in bufs (live runtime tensors)
    std::vector<Buffer> bufs;
    std::vector<std::vector<int32_t>> scopes;  // buffer indices per open scope
    std::multimap<size_t, FreeBlock> free_blocks;
    std::vector<Chunk> chunks;
    size_t chunk_cursor = 0;
    uint64_t record_next = kRecordBase;
    std::unordered_map<uint64_t, HostCopy> host_cache;
    // GRAPH mode: tasks [segment_first, end) wait for the next launch; one
    // cached executable graph per segment index, replayed across runs
    int32_t segment = 0;
    size_t segment_first = 0;
    std::vector<SegmentCache> cache;
    StepSnapshot replay;
    uint64_t replays = 0;
    std::vector<CustomKernel> custom;
    std::vector<std::pair<std::string, hipModule_t>> modules;

    SimplerHipTaskGraph() {
        for (int i = 0; i < kMaxFuncIds; ++i) func_kernel[i] = -1;
    }
};

namespace {

bool device_mode(const SimplerHipTaskGraph *g) { return g->mode != SIMPLER_HIP_TG_RECORD_ONLY; }

int sync_stream(SimplerHipTaskGraph *g) {
    if (!device_mode(g)) return SIMPLER_HIP_OK;
    return hipStreamSynchronize(g->stream) == hipSuccess ? SIMPLER_HIP_OK : SIMPLER_HIP_ERR_LAUNCH;
}

// Device memory for one runtime tensor; *retire receives the tasks that must
// finish before the memory may be written again.
int arena_alloc(SimplerHipTaskGraph *g, size_t bytes, uint64_t *addr, std::vector<int32_t> *retire) {
    const size_t need = (bytes + kAlign - 1) / kAlign * kAlign;
    auto it = g->free_blocks.lower_bound(need);
    if (it != g->free_blocks.end() && it->first <= 2 * need) {
        *addr = it->second.addr;
        *retire = std::move(it->second.retire);
        g->free_blocks.erase(it);
        return SIMPLER_HIP_OK;
    }
    retire->clear();
    if (!device_mode(g)) {
        *addr = g->record_next;
        g->record_next += need;
        return SIMPLER_HIP_OK;
    }
    while (g->chunk_cursor < g->chunks.size()) {
        Chunk &c = g->chunks[g->chunk_cursor];
        if (c.bytes - c.used >= need) {
            *addr = (uint64_t)(uintptr_t)c.base + c.used;
            c.used += need;
            return SIMPLER_HIP_OK;
        }
        ++g->chunk_cursor;
    }
    Chunk c{nullptr, need > kChunkBytes ? need : kChunkBytes, 0};
    if (hipMalloc(&c.base, c.bytes) != hipSuccess) {
        tg_log("device allocation of %zu bytes failed", c.bytes);
        return SIMPLER_HIP_ERR_WORKSPACE;
    }
    c.used = need;
    *addr = (uint64_t)(uintptr_t)c.base;
    g->chunks.push_back(c);
    g->chunk_cursor = g->chunks.size() - 1;
    return SIMPLER_HIP_OK;
}

bool in_graph(const SimplerHipTaskGraph *g, uint64_t id) {
    return id != SIMPLER_HIP_TASK_INVALID && (id >> 32) == 0 && (id & 0xffffffffu) < g->tasks.size();
}

// Tasks whose writes a read of `t` must wait for: the creator and every
// overlapping writer region.
void producers_of(const SimplerHipTaskGraph *g, const SimplerChipTensor &t, std::vector<int32_t> *out) {
    if (in_graph(g, t.owner_task_id)) out->push_back((int32_t)t.owner_task_id);
    auto it = g->tmap.find(t.buffer.addr);
    if (it == g->tmap.end()) return;
    for (const Region &r : it->second)
        if (overlap(r, t) != Overlap::kNone) out->push_back(r.producer);
}

hipKernelNodeParams node_params(const Task &t, void **args) {
    args[0] = const_cast<unsigned char *>(t.launch.data());
    hipKernelNodeParams p{};
    p.func = const_cast<void *>(t.launch.func);
    p.gridDim = t.launch.grid;
    p.blockDim = t.launch.block;
    p.sharedMemBytes = 0;
    p.kernelParams = args;
    p.extra = nullptr;
    return p;
}

// Same kernel, launch shape and in-segment edges: the cached executable graph
// can be replayed after patching the parameter blocks that changed.
bool same_shape(const SegmentCache &c, const SimplerHipTaskGraph *g, size_t first, size_t n) {
    if (c.sigs.size() != n) return false;
    for (size_t i = 0; i < n; ++i) {
        const Task &t = g->tasks[first + i];
        const NodeSig &s = c.sigs[i];
        if (s.func != t.launch.func || s.param_bytes != t.launch.param_bytes || s.grid != t.launch.grid.x ||
            s.block != t.launch.block.x)
            return false;
        size_t k = 0;
        for (int32_t f : t.fanin) {
            if ((size_t)f < first) continue;  // finished in an earlier segment
            if (k >= s.deps.size() || s.deps[k] != (int32_t)((size_t)f - first)) return false;
            ++k;
        }
        if (k != s.deps.size()) return false;
    }
    return true;
}

int build_segment(SegmentCache &c, SimplerHipTaskGraph *g, size_t first, size_t n) {
    c.clear();
    if (hipGraphCreate(&c.graph, 0) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    c.nodes.resize(n);
    c.sigs.resize(n);
    c.params.resize(n);
    std::vector<hipGraphNode_t> deps;
    for (size_t i = 0; i < n; ++i) {
        const Task &t = g->tasks[first + i];
        NodeSig &s = c.sigs[i];
        s.func = t.launch.func;
        s.param_bytes = t.launch.param_bytes;
        s.grid = t.launch.grid.x;
        s.block = t.launch.block.x;
        deps.clear();
        for (int32_t f : t.fanin)
            if ((size_t)f >= first) s.deps.push_back((int32_t)((size_t)f - first));
        if (i > 0) deps.push_back(c.nodes[i - 1]);  // one chain in submission order
        hipError_t e;
        if (t.kernel < 0) {
            e = hipGraphAddEmptyNode(&c.nodes[i], c.graph, deps.data(), deps.size());
        } else {
            void *args[1];
            const hipKernelNodeParams p = node_params(t, args);
            e = hipGraphAddKernelNode(&c.nodes[i], c.graph, deps.data(), deps.size(), &p);
            c.params[i].assign(t.launch.data(), t.launch.data() + t.launch.param_bytes);
        }
        if (e != hipSuccess) {
            tg_log("adding graph node failed: %s", hipGetErrorString(e));
            c.clear();
            return SIMPLER_HIP_ERR_LAUNCH;
        }
    }
    if (hipGraphInstantiate(&c.exec, c.graph, nullptr, nullptr, 0) != hipSuccess) {
        tg_log("hipGraphInstantiate failed");
        c.clear();
        return SIMPLER_HIP_ERR_LAUNCH;
    }
    return SIMPLER_HIP_OK;
}

// GRAPH mode: run the tasks submitted since the last launch as one hipGraph.
int launch_segment(SimplerHipTaskGraph *g) {
    if (g->mode != SIMPLER_HIP_TG_GRAPH) return SIMPLER_HIP_OK;
    const size_t first = g->segment_first, n = g->tasks.size() - first;
    if (n == 0) return SIMPLER_HIP_OK;
    if ((size_t)g->segment >= g->cache.size()) g->cache.resize(g->segment + 1);
    SegmentCache &c = g->cache[g->segment];
    if (c.exec && same_shape(c, g, first, n)) {
        for (size_t i = 0; i < n; ++i) {
            const Task &t = g->tasks[first + i];
            if (t.kernel < 0 || memcmp(c.params[i].data(), t.launch.data(), t.launch.param_bytes) == 0) continue;
            void *args[1];
            const hipKernelNodeParams p = node_params(t, args);
            if (hipGraphExecKernelNodeSetParams(c.exec, c.nodes[i], &p) != hipSuccess) {
                (void)hipGetLastError();
                c.clear();
                break;
            }
            c.params[i].assign(t.launch.data(), t.launch.data() + t.launch.param_bytes);
        }
    }
    if (!c.exec || !same_shape(c, g, first, n)) {
        const int rc = build_segment(c, g, first, n);
        if (rc != SIMPLER_HIP_OK) return rc;
    }
    if (hipGraphLaunch(c.exec, g->stream) != hipSuccess) {
        tg_log("hipGraphLaunch failed");
        return SIMPLER_HIP_ERR_LAUNCH;
    }
    g->segment_first = g->tasks.size();
    ++g->segment;
    return SIMPLER_HIP_OK;
}

// A task writes the buffer at `addr`: its host copy is stale.
void invalidate_host_copy(SimplerHipTaskGraph *g, uint64_t addr) {
    auto it = g->host_cache.find(addr);
    if (it != g->host_cache.end()) it->second.valid = false;
}

// Mark every host copy stale, keeping the pinned buffers for the next step's
// reads of the same tensors; free them all (`release`, or when more than 32
// buffers have accumulated).
void drop_host_copies(SimplerHipTaskGraph *g, bool release) {
    release = release || g->host_cache.size() > 32;
    for (auto &kv : g->host_cache) {
        kv.second.valid = false;
        if (release && kv.second.data) (void)hipHostFree(kv.second.data);
    }
    if (release) g->host_cache.clear();
}

// Queue the copy of external tensor t's bytes into its pinned host copy,
// unless that copy is current (*queued = false). Stream order makes the copy
// follow the work queued so far; the caller's synchronisation then waits for
// both and marks the copy valid.
int queue_host_copy(SimplerHipTaskGraph *g, const SimplerChipTensor &t, HostCopy **out, bool *queued) {
    uint64_t b, e;
    byte_range(t, &b, &e);
    HostCopy &hc = g->host_cache[t.buffer.addr];
    *out = &hc;
    *queued = false;
    if (hc.valid && hc.begin <= b && e <= hc.end) return SIMPLER_HIP_OK;
    hc.valid = false;
    if (hc.cap < e - b) {
        if (hc.data) (void)hipHostFree(hc.data);
        hc.data = nullptr;
        hc.cap = 0;
        void *p = nullptr;
        if (hipHostMalloc(&p, e - b, hipHostMallocDefault) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
        hc.data = static_cast<uint8_t *>(p);
        hc.cap = e - b;
    }
    if (hipMemcpyAsync(hc.data, (const void *)(uintptr_t)(t.buffer.addr + b), e - b, hipMemcpyDeviceToHost,
                       g->stream) != hipSuccess)
        return SIMPLER_HIP_ERR_LAUNCH;
    hc.begin = b;
    hc.end = e;
    *queued = true;
    return SIMPLER_HIP_OK;
}

// Make every task submitted so far complete (used before reading data).
int drain(SimplerHipTaskGraph *g) {
    int rc = launch_segment(g);
    if (rc != SIMPLER_HIP_OK) return rc;
    return sync_stream(g);
}

bool is_custom(int32_t kernel) { return kernel >= kCustomBase; }

// Launch record of a registered kernel: the task's tensors as views, then its
// scalars, in one SimplerHipKernelArgs; the grid from the shape rule.
int make_custom_launch(const SimplerHipTaskGraph *g, int32_t kernel, const SimplerChipTensor *tensors, int32_t n,
                       const uint64_t *scalars, int32_t ns, KernelLaunch *out, char *why, size_t why_len) {
    const CustomKernel &k = g->custom[(size_t)(kernel - kCustomBase)];
    if (n > SIMPLER_HIP_TG_KERNEL_MAX_TENSORS) {
        snprintf(why, why_len, "%d tensors, at most %d for a registered kernel", n, SIMPLER_HIP_TG_KERNEL_MAX_TENSORS);
        return SIMPLER_HIP_ERR_INVALID;
    }
    if (k.grid_tensor >= n) {
        snprintf(why, why_len, "the kernel's grid follows tensor %d, but the task has %d", k.grid_tensor, n);
        return SIMPLER_HIP_ERR_INVALID;
    }
    SimplerHipKernelArgs a;
    memset(&a, 0, sizeof(a));
    a.n_tensors = n;
    a.n_scalars = ns;
    for (int i = 0; i < n; ++i) {
        const SimplerChipTensor &t = tensors[i];
        SimplerHipKernelTensor &v = a.tensors[i];
        v.addr = t.buffer.addr + t.start_offset * simpler_dtype_size(t.dtype);
        v.ndims = t.ndims;
        v.dtype = t.dtype;
        for (uint32_t d = 0; d < t.ndims; ++d) {
            v.shapes[d] = t.shapes[d];
            v.strides[d] = t.strides[d];
        }
    }
    for (int i = 0; i < ns; ++i) a.scalars[i] = scalars[i];
    uint64_t grid = k.per_wg;
    if (k.grid_tensor >= 0) grid = (numel(tensors[k.grid_tensor]) + k.per_wg - 1) / k.per_wg;
    if (grid == 0) grid = 1;
    if (grid > 0x7fffffffu) {
        snprintf(why, why_len, "grid of %llu workgroups", (unsigned long long)grid);
        return SIMPLER_HIP_ERR_INVALID;
    }
    out->func = reinterpret_cast<const void *>(k.fn);
    out->grid = dim3((unsigned)grid, 1, 1);
    out->block = dim3(k.block, 1, 1);
    out->param_bytes = sizeof(a);
    const unsigned char *ab = reinterpret_cast<const unsigned char *>(&a);
    out->big.assign(ab, ab + sizeof(a));
    return SIMPLER_HIP_OK;
}

int make_launch(const SimplerHipTaskGraph *g, int32_t kernel, const SimplerChipTensor *tensors, int32_t n,
                const uint64_t *scalars, int32_t ns, KernelLaunch *out, char *why, size_t why_len) {
    if (is_custom(kernel)) return make_custom_launch(g, kernel, tensors, n, scalars, ns, out, why, why_len);
    return simpler_hip::make_incore_launch(kernel, tensors, n, scalars, ns, out, why, why_len);
}

// EAGER: launch now. GRAPH: the task waits in the segment until launch.
int record_task(SimplerHipTaskGraph *g, Task &t) {
    if (g->mode != SIMPLER_HIP_TG_EAGER || t.kernel < 0) return SIMPLER_HIP_OK;
    void *args[1] = {const_cast<unsigned char *>(t.launch.data())};
    hipError_t e;
    if (is_custom(t.kernel))
        e = hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(const_cast<void *>(t.launch.func)), t.launch.grid.x,
                                  1, 1, t.launch.block.x, 1, 1, 0, g->stream, args, nullptr);
    else
        e = hipLaunchKernel(t.launch.func, t.launch.grid, t.launch.block, args, 0, g->stream);
    if (e != hipSuccess) {
        tg_log("launch of kernel %d failed: %s", t.kernel, hipGetErrorString(e));
        (void)hipGetLastError();
        return SIMPLER_HIP_ERR_LAUNCH;
    }
    return SIMPLER_HIP_OK;
}

SimplerChipTensor materialize(const SimplerChipTensor &ci, uint64_t addr, size_t bytes, int32_t owner) {
    SimplerChipTensor t;
    memset(&t, 0, sizeof(t));
    t.buffer.addr = addr;
    t.buffer.size = bytes;
    t.owner_task_id = (uint64_t)owner;
    t.ndims = ci.ndims;
    t.dtype = ci.dtype;
    t.is_contiguous = 1;
    t.address_space = SIMPLER_ADDR_DEVICE;
    uint64_t acc = 1;
    for (int d = (int)ci.ndims - 1; d >= 0; --d) {
        t.shapes[d] = ci.shapes[d];
        t.strides[d] = (uint32_t)acc;
        acc *= ci.shapes[d];
    }
    t.extent_elem_cache = acc;
    return t;
}

}  // namespace

int32_t simpler_hip::tg_mode_of(const SimplerHipTaskGraph *g) { return g->mode; }

int simpler_hip::tg_prefetch_host(SimplerHipTaskGraph *g, const SimplerChipTensor *tensors, int n) {
    if (!device_mode(g)) return SIMPLER_HIP_OK;
    std::vector<HostCopy *> pending;
    for (int i = 0; i < n; ++i) {
        const SimplerChipTensor &t = tensors[i];
        if (t.address_space != SIMPLER_ADDR_DEVICE || !valid_tensor(t)) continue;
        std::vector<int32_t> prod;
        producers_of(g, t, &prod);
        if (!prod.empty()) continue;  // written by this graph's tasks: read after they finish
        HostCopy *hc = nullptr;
        bool queued = false;
        const int rc = queue_host_copy(g, t, &hc, &queued);
        if (rc != SIMPLER_HIP_OK) return rc;
        if (queued) pending.push_back(hc);
    }
    if (pending.empty()) return SIMPLER_HIP_OK;
    if (hipStreamSynchronize(g->stream) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
    for (HostCopy *hc : pending) hc->valid = true;
    return SIMPLER_HIP_OK;
}

bool simpler_hip::tg_is_fresh(const SimplerHipTaskGraph *g) {
    if (!g->tasks.empty() || g->segment != 0 || g->segment_first != 0 || !g->free_blocks.empty() ||
        !g->bufs.empty() || g->chunk_cursor != 0)
        return false;
    for (const auto &sc : g->scopes)  // scopes may be open, but hold nothing yet
        if (!sc.empty()) return false;
    for (const Chunk &c : g->chunks)
        if (c.used) return false;
    return true;
}

extern "C" {

SimplerHipTaskGraph *simpler_hip_tg_create(int32_t mode, void *stream) {
    if (mode != SIMPLER_HIP_TG_EAGER && mode != SIMPLER_HIP_TG_GRAPH && mode != SIMPLER_HIP_TG_RECORD_ONLY)
        return nullptr;
    SimplerHipTaskGraph *g = new (std::nothrow) SimplerHipTaskGraph();
    if (!g) return nullptr;
    g->mode = mode;
    g->stream = static_cast<hipStream_t>(stream);
    if (mode != SIMPLER_HIP_TG_RECORD_ONLY && hipGetDevice(&g->device) != hipSuccess) {
        delete g;
        return nullptr;
    }
    return g;
}

void simpler_hip_tg_destroy(SimplerHipTaskGraph *g) {
    if (!g) return;
    if (device_mode(g)) {
        sync_stream(g);
        for (SegmentCache &c : g->cache) c.clear();
        for (Chunk &c : g->chunks) (void)hipFree(c.base);
        for (auto &m : g->modules) (void)hipModuleUnload(m.second);
        drop_host_copies(g, true);
    }
    delete g;
}

int simpler_hip_tg_bind(SimplerHipTaskGraph *g, int32_t func_id, int32_t kernel) {
    if (!g || func_id < 0 || func_id >= kMaxFuncIds || simpler_hip::incore_tensor_count(kernel) < 0)
        return SIMPLER_HIP_ERR_INVALID;
    g->func_kernel[func_id] = kernel;
    return SIMPLER_HIP_OK;
}

int simpler_hip_tg_register_kernel(SimplerHipTaskGraph *g, int32_t func_id, const char *code_object_path,
                                   const char *kernel_name, uint32_t block_threads, int32_t grid_tensor,
                                   uint32_t elems_per_workgroup) {
    if (!g || func_id < 0 || func_id >= kMaxFuncIds || !code_object_path || !kernel_name || block_threads == 0 ||
        block_threads > 1024 || elems_per_workgroup == 0 || grid_tensor >= SIMPLER_HIP_TG_KERNEL_MAX_TENSORS) {
        tg_log("register_kernel: bad argument");
        return SIMPLER_HIP_ERR_INVALID;
    }
    if (g->custom.size() >= (size_t)kMaxFuncIds * 4) return SIMPLER_HIP_ERR_INVALID;
    CustomKernel k;
    k.block = block_threads;
    k.grid_tensor = grid_tensor < 0 ? -1 : grid_tensor;
    k.per_wg = elems_per_workgroup;
    if (device_mode(g)) {
        hipModule_t mod = nullptr;
        for (auto &m : g->modules)
            if (m.first == code_object_path) mod = m.second;
        if (!mod) {
            int cur = -1;
            if (hipGetDevice(&cur) != hipSuccess || (cur != g->device && hipSetDevice(g->device) != hipSuccess))
                return SIMPLER_HIP_ERR_LAUNCH;
            const hipError_t e = hipModuleLoad(&mod, code_object_path);
            if (cur != g->device) (void)hipSetDevice(cur);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                tg_log("register_kernel: cannot load code object %s: %s", code_object_path, hipGetErrorString(e));
                return SIMPLER_HIP_ERR_UNSUPPORTED;
            }
            g->modules.emplace_back(code_object_path, mod);
        }
        if (hipModuleGetFunction(&k.fn, mod, kernel_name) != hipSuccess) {
            (void)hipGetLastError();
            tg_log("register_kernel: no kernel %s in %s", kernel_name, code_object_path);
            return SIMPLER_HIP_ERR_UNSUPPORTED;
        }
    }
    g->custom.push_back(k);
    g->func_kernel[func_id] = kCustomBase + (int32_t)(g->custom.size() - 1);
    return SIMPLER_HIP_OK;
}

int simpler_hip_tg_scope_begin(SimplerHipTaskGraph *g) {
    if (!g) return SIMPLER_HIP_ERR_INVALID;
    g->scopes.emplace_back();
    return SIMPLER_HIP_OK;
}

int simpler_hip_tg_scope_end(SimplerHipTaskGraph *g) {
    if (!g || g->scopes.empty()) return SIMPLER_HIP_ERR_INVALID;
    for (int32_t bi : g->scopes.back()) {
        Buffer &b = g->bufs[bi];
        g->tmap.erase(b.addr);
        g->buf_of.erase(b.addr);
        invalidate_host_copy(g, b.addr);
        FreeBlock fb{b.addr, (b.bytes + kAlign - 1) / kAlign * kAlign, std::move(b.users)};
        g->free_blocks.emplace(fb.bytes, std::move(fb));
        b.users.clear();
    }
    g->scopes.pop_back();
    return SIMPLER_HIP_OK;
}

int64_t simpler_hip_tg_submit(SimplerHipTaskGraph *g, int32_t func_id, const SimplerChipTensor *tensors,
                              const int32_t *arg_types, int32_t n, const uint64_t *scalars, int32_t ns,
                              const uint64_t *explicit_deps, int32_t nd, SimplerChipTensor *outputs) {
    if (!g || n < 0 || n > SIMPLER_CORE_MAX_TENSOR_ARGS || ns < 0 || ns > SIMPLER_CORE_MAX_SCALAR_ARGS || nd < 0 ||
        (n > 0 && (!tensors || !arg_types)) || (ns > 0 && !scalars) || (nd > 0 && !explicit_deps)) {
        tg_log("submit: bad argument counts or pointers");
        return SIMPLER_HIP_ERR_INVALID;
    }
    if (g->tasks.size() >= 0x7fffffff) return SIMPLER_HIP_ERR_INVALID;
    int32_t kernel = -1;
    if (func_id >= 0) {
        if (func_id >= kMaxFuncIds || g->func_kernel[func_id] < 0) {
            tg_log("submit: func_id %d is not bound to a kernel", func_id);
            return SIMPLER_HIP_ERR_UNSUPPORTED;
        }
        kernel = g->func_kernel[func_id];
    }
    const int32_t id = (int32_t)g->tasks.size();
    for (int i = 0; i < n; ++i) {
        const int32_t ty = arg_types[i];
        if (ty < SIMPLER_HIP_TA_INPUT || ty > SIMPLER_HIP_TA_NO_DEP || !valid_tensor(tensors[i])) {
            tg_log("submit: tensor %d has a bad tag, ndims, dtype or stride", i);
            return SIMPLER_HIP_ERR_INVALID;
        }
        if (kernel >= 0 && ty != SIMPLER_HIP_TA_OUTPUT && device_mode(g) &&
            tensors[i].address_space != SIMPLER_ADDR_DEVICE) {
            tg_log("submit: tensor %d is host memory; kernels read device memory only", i);
            return SIMPLER_HIP_ERR_INVALID;
        }
    }
    for (int i = 0; i < nd; ++i)
        if (!in_graph(g, explicit_deps[i])) {
            tg_log("submit: explicit dependency %llu is not a task of this graph",
                   (unsigned long long)explicit_deps[i]);
            return SIMPLER_HIP_ERR_INVALID;
        }

    // Dry run of the kernel's argument check with placeholder outputs, so a
    // rejected task leaves no trace in the graph.
    std::vector<SimplerChipTensor> args(tensors, tensors + n);
    if (kernel >= 0) {
        std::vector<SimplerChipTensor> probe(args);
        for (int i = 0; i < n; ++i)
            if (arg_types[i] == SIMPLER_HIP_TA_OUTPUT)
                probe[i] = materialize(args[i], kRecordBase, numel(args[i]) * simpler_dtype_size(args[i].dtype), id);
        KernelLaunch tmp;
        char why[256] = {};
        const int rc = make_launch(g, kernel, probe.data(), n, scalars, ns, &tmp, why, sizeof(why));
        if (rc != SIMPLER_HIP_OK) {
            tg_log("submit: func_id %d: %s", func_id, why);
            return rc;
        }
    }

    Task t;
    t.func_id = func_id;
    t.kernel = kernel;
    std::vector<int32_t> &fanin = t.fanin;
    for (int i = 0; i < nd; ++i) fanin.push_back((int32_t)(explicit_deps[i] & 0xffffffffu));

    // creator edges and TensorMap lookups
    for (int i = 0; i < n; ++i) {
        const int32_t ty = arg_types[i];
        if (ty == SIMPLER_HIP_TA_OUTPUT) continue;
        const SimplerChipTensor &x = args[i];
        if (in_graph(g, x.owner_task_id)) fanin.push_back((int32_t)x.owner_task_id);
        if ((ty != SIMPLER_HIP_TA_INPUT && ty != SIMPLER_HIP_TA_INOUT) || x.manual_dep) continue;
        auto it = g->tmap.find(x.buffer.addr);
        if (it == g->tmap.end()) continue;
        std::vector<Region> &regs = it->second;
        for (size_t k = 0; k < regs.size();) {
            const Overlap ov = overlap(regs[k], x);
            if (ov != Overlap::kNone) {
                fanin.push_back(regs[k].producer);
                if (ty == SIMPLER_HIP_TA_INOUT && ov == Overlap::kCovered) {  // superseded writer: retire
                    regs[k] = regs.back();
                    regs.pop_back();
                    continue;
                }
            }
            ++k;
        }
    }

    // runtime-allocated outputs
    for (int i = 0; i < n; ++i) {
        if (arg_types[i] != SIMPLER_HIP_TA_OUTPUT) continue;
        const size_t bytes = numel(args[i]) * simpler_dtype_size(args[i].dtype);
        uint64_t addr = 0;
        std::vector<int32_t> retire;
        const int rc = arena_alloc(g, bytes ? bytes : 1, &addr, &retire);
        if (rc != SIMPLER_HIP_OK) return rc;
        fanin.insert(fanin.end(), retire.begin(), retire.end());
        args[i] = materialize(args[i], addr, bytes, id);
        const int32_t bi = (int32_t)g->bufs.size();
        g->bufs.push_back(Buffer{addr, bytes, {id}});
        g->buf_of[addr] = bi;
        if (!g->scopes.empty()) g->scopes.back().push_back(bi);
        g->tmap.erase(addr);  // fresh tensor at recycled memory: no older writers
    }

    // users of runtime tensors (for write-after-read on reuse)
    for (int i = 0; i < n; ++i) {
        if (arg_types[i] == SIMPLER_HIP_TA_OUTPUT) continue;
        auto it = g->buf_of.find(args[i].buffer.addr);
        if (it != g->buf_of.end()) g->bufs[it->second].users.push_back(id);
    }

    // publish writers
    for (int i = 0; i < n; ++i) {
        const int32_t ty = arg_types[i];
        if ((ty != SIMPLER_HIP_TA_INOUT && ty != SIMPLER_HIP_TA_OUTPUT_EXISTING) || args[i].manual_dep) continue;
        g->tmap[args[i].buffer.addr].push_back(region_of(args[i], id));
        invalidate_host_copy(g, args[i].buffer.addr);
    }

    std::sort(fanin.begin(), fanin.end());
    fanin.erase(std::unique(fanin.begin(), fanin.end()), fanin.end());

    if (kernel >= 0) {
        char why[256] = {};
        const int rc = make_launch(g, kernel, args.data(), n, scalars, ns, &t.launch, why, sizeof(why));
        if (rc != SIMPLER_HIP_OK) {  // not reached: the dry run accepted the same shapes
            tg_log("submit: func_id %d: %s", func_id, why);
            return rc;
        }
    }
    g->tasks.push_back(std::move(t));
    const int rc = record_task(g, g->tasks.back());
    if (rc != SIMPLER_HIP_OK) return rc;
    if (outputs)
        for (int i = 0; i < n; ++i) outputs[i] = args[i];
    return id;
}

int64_t simpler_hip_tg_alloc(SimplerHipTaskGraph *g, const SimplerChipTensor *create_infos, int32_t n,
                             SimplerChipTensor *outputs) {
    if (!g || n <= 0 || n > SIMPLER_CORE_MAX_TENSOR_ARGS || !create_infos) return SIMPLER_HIP_ERR_INVALID;
    std::vector<int32_t> tags(n, SIMPLER_HIP_TA_OUTPUT);
    return simpler_hip_tg_submit(g, -1, create_infos, tags.data(), n, nullptr, 0, nullptr, 0, outputs);
}

int simpler_hip_tg_get_tensor_data(SimplerHipTaskGraph *g, const SimplerChipTensor *t, uint32_t ndims,
                                   const uint32_t *idx, uint64_t *value) {
    if (!g || !t || !value || !valid_tensor(*t) || ndims != t->ndims || (ndims && !idx))
        return SIMPLER_HIP_ERR_INVALID;
    uint64_t off = t->start_offset;
    for (uint32_t d = 0; d < ndims; ++d) {
        if (idx[d] >= t->shapes[d]) {
            tg_log("get_tensor_data: index %u out of range in dim %u (size %u)", idx[d], d, t->shapes[d]);
            return SIMPLER_HIP_ERR_INVALID;
        }
        off += (uint64_t)idx[d] * t->strides[d];
    }
    const uint64_t esz = simpler_dtype_size(t->dtype);
    uint64_t v = 0;
    if (t->address_space == SIMPLER_ADDR_HOST) {
        memcpy(&v, (const void *)(uintptr_t)(t->buffer.addr + off * esz), esz);
        *value = v;
        return SIMPLER_HIP_OK;
    }
    if (!device_mode(g)) return SIMPLER_HIP_ERR_UNSUPPORTED;
    std::vector<int32_t> prod;
    producers_of(g, *t, &prod);
    if (!prod.empty()) {  // written inside this graph: finish the writers, read fresh
        int rc = drain(g);
        if (rc != SIMPLER_HIP_OK) return rc;
        if (hipMemcpy(&v, (const void *)(uintptr_t)(t->buffer.addr + off * esz), esz, hipMemcpyDeviceToHost) !=
            hipSuccess)
            return SIMPLER_HIP_ERR_LAUNCH;
        *value = v;
        return SIMPLER_HIP_OK;
    }
    // external input: one copy of the view's extent, reused until a task writes the buffer
    uint64_t b, e;
    byte_range(*t, &b, &e);
    HostCopy *hc = nullptr;
    bool queued = false;
    int rc = queue_host_copy(g, *t, &hc, &queued);
    if (rc != SIMPLER_HIP_OK) return rc;
    if (queued) {
        if (hipStreamSynchronize(g->stream) != hipSuccess) return SIMPLER_HIP_ERR_LAUNCH;
        hc->valid = true;
    }
    memcpy(&v, hc->data + (off * esz - hc->begin), esz);
    *value = v;
    return SIMPLER_HIP_OK;
}

int simpler_hip_tg_copy_to_host(SimplerHipTaskGraph *g, const SimplerChipTensor *t, void *host, uint64_t bytes) {
    if (!g || !t || !host || !valid_tensor(*t)) return SIMPLER_HIP_ERR_INVALID;
    uint64_t b, e;
    byte_range(*t, &b, &e);
    if (bytes < e - b) return SIMPLER_HIP_ERR_INVALID;
    if (t->address_space == SIMPLER_ADDR_HOST) {
        memcpy(host, (const void *)(uintptr_t)(t->buffer.addr + b), e - b);
        return SIMPLER_HIP_OK;
    }
    if (!device_mode(g)) return SIMPLER_HIP_ERR_UNSUPPORTED;
    const int rc = drain(g);
    if (rc != SIMPLER_HIP_OK) return rc;
    if (e == b) return SIMPLER_HIP_OK;
    return hipMemcpy(host, (const void *)(uintptr_t)(t->buffer.addr + b), e - b, hipMemcpyDeviceToHost) == hipSuccess
               ? SIMPLER_HIP_OK
               : SIMPLER_HIP_ERR_LAUNCH;
}

int simpler_hip_tg_launch(SimplerHipTaskGraph *g) {
    if (!g) return SIMPLER_HIP_ERR_INVALID;
    return launch_segment(g);
}

int simpler_hip_tg_wait(SimplerHipTaskGraph *g) {
    if (!g) return SIMPLER_HIP_ERR_INVALID;
    return sync_stream(g);
}

int simpler_hip_tg_reset(SimplerHipTaskGraph *g) {
    if (!g) return SIMPLER_HIP_ERR_INVALID;
    const int rc = sync_stream(g);
    g->tasks.clear();
    g->tmap.clear();
    g->buf_of.clear();
    g->bufs.clear();
    g->scopes.clear();
    g->free_blocks.clear();
    drop_host_copies(g, false);
    for (Chunk &c : g->chunks) c.used = 0;
    g->chunk_cursor = 0;
    g->record_next = kRecordBase;
    g->segment = 0;
    g->segment_first = 0;
    return rc;
}

int simpler_hip_tg_record_replay(SimplerHipTaskGraph *g, const void *key, uint64_t key_bytes) {
    if (!g || (key_bytes && !key)) return SIMPLER_HIP_ERR_INVALID;
    if (g->mode != SIMPLER_HIP_TG_GRAPH) return SIMPLER_HIP_OK;
    if (g->segment != 0 || g->segment_first != 0) {
        tg_log("record_replay: the step has launched work");
        return SIMPLER_HIP_ERR_INVALID;
    }
    StepSnapshot &r = g->replay;
    r.valid = false;
    const uint8_t *kb = static_cast<const uint8_t *>(key);
    r.key.assign(kb, kb + key_bytes);
    r.tasks = g->tasks;
    r.tmap = g->tmap;
    r.buf_of = g->buf_of;
    r.bufs = g->bufs;
    r.scopes = g->scopes;
    r.free_blocks = g->free_blocks;
    r.chunk_used.clear();
    for (const Chunk &c : g->chunks) r.chunk_used.push_back(c.used);
    r.chunk_cursor = g->chunk_cursor;
    r.record_next = g->record_next;
    r.valid = true;
    return SIMPLER_HIP_OK;
}

int simpler_hip_tg_replay(SimplerHipTaskGraph *g, const void *key, uint64_t key_bytes) {
    if (!g || (key_bytes && !key)) return SIMPLER_HIP_ERR_INVALID;
    const StepSnapshot &r = g->replay;
    if (g->mode != SIMPLER_HIP_TG_GRAPH || !r.valid || r.key.size() != key_bytes ||
        (key_bytes && memcmp(r.key.data(), key, key_bytes) != 0) || r.chunk_used.size() > g->chunks.size() ||
        r.scopes.size() != g->scopes.size() || !simpler_hip::tg_is_fresh(g))
        return 0;
    g->tasks = r.tasks;
    g->tmap = r.tmap;
    g->buf_of = r.buf_of;
    g->bufs = r.bufs;
    g->scopes = r.scopes;
    g->free_blocks = r.free_blocks;
    for (size_t i = 0; i < g->chunks.size(); ++i) g->chunks[i].used = i < r.chunk_used.size() ? r.chunk_used[i] : 0;
    g->chunk_cursor = r.chunk_cursor;
    g->record_next = r.record_next;
    ++g->replays;
    return 1;
}

int64_t simpler_hip_tg_task_count(const SimplerHipTaskGraph *g) { return g ? (int64_t)g->tasks.size() : -1; }

uint64_t simpler_hip_tg_replay_count(const SimplerHipTaskGraph *g) { return g ? g->replays : 0; }

int32_t simpler_hip_tg_fanin(const SimplerHipTaskGraph *g, int64_t task, int64_t *producers, int32_t cap) {
    if (!g || task < 0 || task >= (int64_t)g->tasks.size()) return SIMPLER_HIP_ERR_INVALID;
    const std::vector<int32_t> &f = g->tasks[task].fanin;
    for (int32_t i = 0; i < cap && i < (int32_t)f.size(); ++i) producers[i] = f[i];
    return (int32_t)f.size();
}

uint64_t simpler_hip_tg_arena_bytes(const SimplerHipTaskGraph *g) {
    if (!g) return 0;
    uint64_t s = 0;
    for (const Chunk &c : g->chunks) s += c.bytes;
    return s;
}

}  // extern "C"
