// MLA decode kernels (Dk 576, Dv 512, V a prefix of K; bf16): block sizes 32
// and 64, fp32 or bf16 output. The fused KV append runs as a launch of its own
// ahead of these (simpler_hip_pa_decode_append).
#include "pa_kernels.h"

namespace simpler_hip {
namespace pa {

KernelPair pick_mla(int bs, int out_dtype) {
    const bool f32 = out_dtype == SIMPLER_HIP_DT_FLOAT32, b16 = out_dtype == SIMPLER_HIP_DT_BFLOAT16;
    if (bs == 32 && f32) return {pa_mla_kernel<32, kMlaDk, kMlaDv, float>, nullptr, true, false};
    if (bs == 32 && b16) return {pa_mla_kernel<32, kMlaDk, kMlaDv, __bf16>, nullptr, true, false};
    if (bs == 64 && f32) return {pa_mla_kernel<64, kMlaDk, kMlaDv, float>, nullptr, true, false};
    if (bs == 64 && b16) return {pa_mla_kernel<64, kMlaDk, kMlaDv, __bf16>, nullptr, true, false};
    return KernelPair{};
}

}  // namespace pa
}  // namespace simpler_hip
