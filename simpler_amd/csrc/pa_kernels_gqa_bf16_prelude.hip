// GQA decode kernels with the fused KV append and the fused decode prelude:
// bf16 caches, 128-dim heads (fp32 or bf16 output).
#include "pa_kernels_gqa.h"

namespace simpler_hip {
namespace pa {

KernelPair pick_gqa_bf16_prelude(int bs, int d, int out_dtype) {
    if (out_dtype == SIMPLER_HIP_DT_FLOAT32) return prelude_by_block<float>(bs, d);
    if (out_dtype == SIMPLER_HIP_DT_BFLOAT16) return prelude_by_block<__bf16>(bs, d);
    return KernelPair{};
}

}  // namespace pa
}  // namespace simpler_hip
