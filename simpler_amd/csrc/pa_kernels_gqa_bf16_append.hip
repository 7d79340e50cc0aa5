// GQA decode kernels with the fused KV append: bf16 query and caches (fp32 or bf16 output).
#include "pa_kernels_gqa.h"

namespace simpler_hip {
namespace pa {

KernelPair pick_gqa_bf16_append(int bs, int d, int out_dtype) {
    if (out_dtype == SIMPLER_HIP_DT_FLOAT32) return gqa_by_block<float, __bf16, true>(bs, d);
    if (out_dtype == SIMPLER_HIP_DT_BFLOAT16) return gqa_by_block<__bf16, __bf16, true>(bs, d);
    return KernelPair{};
}

}  // namespace pa
}  // namespace simpler_hip
