// GQA decode kernels with the fused KV append: fp16 query and caches (fp32 or fp16 output).
#include "pa_kernels_gqa.h"

namespace simpler_hip {
namespace pa {

KernelPair pick_gqa_f16_append(int bs, int d, int out_dtype) {
    if (out_dtype == SIMPLER_HIP_DT_FLOAT32) return gqa_by_block<float, _Float16, true>(bs, d);
    if (out_dtype == SIMPLER_HIP_DT_FLOAT16) return gqa_by_block<_Float16, _Float16, true>(bs, d);
    return KernelPair{};
}

}  // namespace pa
}  // namespace simpler_hip
