// Incore kernels of the task-graph backend: one HIP kernel per simpler
// AICore/AIV kernel the graph can run, each described to the host as a
// ready-to-launch record (function, grid, block, one by-value parameter
// block) built from the task's ChipTensor arguments.
//
// Internal to libsimpler_hip.so (shared by incore_kernels.hip and
// task_graph.cpp); the public surface is include/simpler_hip/task_graph.h.
#pragma once

#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "simpler_hip/abi_types.h"

namespace simpler_hip {

constexpr size_t kMaxKernelParamBytes = 256;  // built-in kernels' parameter blocks

struct KernelLaunch {
    const void *func = nullptr;  // __global__ function
    dim3 grid{1, 1, 1};
    dim3 block{64, 1, 1};
    size_t param_bytes = 0;
    alignas(16) unsigned char params[kMaxKernelParamBytes] = {};
    std::vector<unsigned char> big;  // a larger parameter block (registered kernels), used instead of params
    const unsigned char *data() const { return big.empty() ? params : big.data(); }
};

// Validates the task's tensors and scalars for `kernel` (a
// SimplerHipIncoreKernel code) and fills `out`. Returns 0, or
// SIMPLER_HIP_ERR_INVALID / SIMPLER_HIP_ERR_UNSUPPORTED with a message in
// `why` (at least 160 bytes).
int make_incore_launch(int32_t kernel, const SimplerChipTensor *tensors, int32_t n_tensors, const uint64_t *scalars,
                       int32_t n_scalars, KernelLaunch *out, char *why, size_t why_len);

// Expected tensor count and argument roles of a kernel (for signature checks):
// returns the tensor count, or -1 for an unknown kernel.
int incore_tensor_count(int32_t kernel);

}  // namespace simpler_hip
