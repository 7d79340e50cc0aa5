// GQA decode kernels with bf16 query and caches (fp32 or bf16 output).
#include "pa_kernels_gqa.h"

namespace simpler_hip {
namespace pa {

KernelPair pick_gqa_bf16(int bs, int d, int out_dtype) {
    if (out_dtype == SIMPLER_HIP_DT_FLOAT32) return gqa_by_block<float, __bf16, false>(bs, d);
    if (out_dtype == SIMPLER_HIP_DT_BFLOAT16) return gqa_by_block<__bf16, __bf16, false>(bs, d);
    return KernelPair{};
}

}  // namespace pa
}  // namespace simpler_hip
