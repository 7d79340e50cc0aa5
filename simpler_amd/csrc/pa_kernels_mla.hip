// MLA decode kernels (Dk 576, Dv 512, V a prefix of K; bf16): block sizes 32
// and 64, fp32 or bf16 output, without or with the fused KV append.
#include "pa_kernels.h"

namespace simpler_hip {
namespace pa {

namespace {
template <bool APPEND>
KernelPair mla_kernels(int bs, int out_dtype) {
    const bool f32 = out_dtype == SIMPLER_HIP_DT_FLOAT32, b16 = out_dtype == SIMPLER_HIP_DT_BFLOAT16;
    if (bs == 32 && f32) return {pa_mla_kernel<32, kMlaDk, kMlaDv, float, APPEND>, nullptr, true, false};
    if (bs == 32 && b16) return {pa_mla_kernel<32, kMlaDk, kMlaDv, __bf16, APPEND>, nullptr, true, false};
    if (bs == 64 && f32) return {pa_mla_kernel<64, kMlaDk, kMlaDv, float, APPEND>, nullptr, true, false};
    if (bs == 64 && b16) return {pa_mla_kernel<64, kMlaDk, kMlaDv, __bf16, APPEND>, nullptr, true, false};
    return KernelPair{};
}
}  // namespace

KernelPair pick_mla(int bs, int out_dtype, bool append) {
    return append ? mla_kernels<true>(bs, out_dtype) : mla_kernels<false>(bs, out_dtype);
}

}  // namespace pa
}  // namespace simpler_hip
