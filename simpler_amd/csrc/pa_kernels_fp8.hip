// GQA decode kernels with fp8 E4M3FN caches and a bf16 query: head dim 128
// (Llama/Qwen GQA), the four block sizes, fp32 or bf16 output.
#include "pa_kernels.h"

namespace simpler_hip {
namespace pa {
namespace {

template <int BS, typename OutT>
KernelPair fp8_pair() {
    return {pa_decode_kernel<BS, 128, 128, OutT, 1, true>, pa_decode_kernel<BS, 128, 128, OutT, kMaxWavesPerWorker, true>,
            false, false};
}

template <typename OutT>
KernelPair fp8_by_block(int bs) {
    switch (bs) {
        case 16: return fp8_pair<16, OutT>();
        case 32: return fp8_pair<32, OutT>();
        case 64: return fp8_pair<64, OutT>();
        case 128: return fp8_pair<128, OutT>();
        default: return KernelPair{};
    }
}

}  // namespace

KernelPair pick_gqa_fp8(int bs, int d, int out_dtype) {
    if (d != 128) return KernelPair{};
    if (out_dtype == SIMPLER_HIP_DT_FLOAT32) return fp8_by_block<float>(bs);
    if (out_dtype == SIMPLER_HIP_DT_BFLOAT16) return fp8_by_block<__bf16>(bs);
    return KernelPair{};
}

}  // namespace pa
}  // namespace simpler_hip
