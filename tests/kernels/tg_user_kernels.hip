// Kernels of a caller's own for the task-graph backend
// (simpler_hip_tg_register_kernel; tests/test_task_graph_gpu.py). Each takes
// the task's tensors, then its scalars, as one SimplerHipKernelArgs, and reads
// tensors through their views (shapes and strides), as a task may pass a view.
#include <hip/hip_runtime.h>

#include "simpler_hip/task_graph.h"

namespace {

__device__ uint64_t numel(const SimplerHipKernelTensor &t) {
    uint64_t n = 1;
    for (uint32_t d = 0; d < t.ndims; ++d) n *= t.shapes[d];
    return n;
}

// Element offset (in elements) of row-major index i within view t.
__device__ uint64_t elem_offset(const SimplerHipKernelTensor &t, uint64_t i) {
    uint64_t off = 0;
    for (int d = (int)t.ndims - 1; d >= 0; --d) {
        off += (i % t.shapes[d]) * t.strides[d];
        i /= t.shapes[d];
    }
    return off;
}

__device__ float &at(const SimplerHipKernelTensor &t, uint64_t i) {
    return reinterpret_cast<float *>(t.addr)[elem_offset(t, i)];
}

}  // namespace

// y = alpha * x + b. Tensors x, b, y: fp32 with the same element count;
// scalar 0: alpha as fp32 bits.
extern "C" __global__ void __launch_bounds__(256) tg_axpb(const SimplerHipKernelArgs a) {
    const SimplerHipKernelTensor &x = a.tensors[0], &b = a.tensors[1], &y = a.tensors[2];
    const float alpha = __uint_as_float((uint32_t)a.scalars[0]);
    const uint64_t n = numel(y);
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        at(y, i) = alpha * at(x, i) + at(b, i);
}

// y[r][c] = x[r][c] * s[r]. x, y: fp32 [R, C]; s: fp32 [R].
extern "C" __global__ void __launch_bounds__(128) tg_row_scale(const SimplerHipKernelArgs a) {
    const SimplerHipKernelTensor &x = a.tensors[0], &s = a.tensors[1], &y = a.tensors[2];
    const uint64_t cols = y.shapes[1], n = numel(y);
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        at(y, i) = at(x, i) * at(s, i / cols);
}
