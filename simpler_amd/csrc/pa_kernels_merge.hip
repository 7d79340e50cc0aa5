// Split-merge kernels (pa_merge_kernel) for every output width and dtype the
// decode kernels produce.
#include "pa_kernels.h"

namespace simpler_hip {
namespace pa {
namespace {

template <int DV>
MergeFn merge_for(int out_dtype) {
    switch (out_dtype) {
        case SIMPLER_HIP_DT_FLOAT32: return {pa_merge_kernel<DV, float>, merge_threads<DV>()};
        case SIMPLER_HIP_DT_BFLOAT16: return {pa_merge_kernel<DV, __bf16>, merge_threads<DV>()};
        case SIMPLER_HIP_DT_FLOAT16: return {pa_merge_kernel<DV, _Float16>, merge_threads<DV>()};
        default: return MergeFn{};
    }
}

}  // namespace

MergeFn pick_merge(int dv, int out_dtype) {
    switch (dv) {
        case 16: return merge_for<16>(out_dtype);
        case 32: return merge_for<32>(out_dtype);
        case 64: return merge_for<64>(out_dtype);
        case 128: return merge_for<128>(out_dtype);
        case 256: return merge_for<256>(out_dtype);
        case kMlaDv: return merge_for<kMlaDv>(out_dtype);
        default: return MergeFn{};
    }
}

}  // namespace pa
}  // namespace simpler_hip
