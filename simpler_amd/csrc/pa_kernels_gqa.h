// Kernel tables of the GQA decode for one element type: every supported
// (block size, head dim) pair of pa_decode_kernel, one wave per worker and up
// to kMaxWavesPerWorker sibling waves, without or with the fused KV append.
// Included by pa_kernels_gqa_{bf16,f16}{,_append}.hip, so each element type
// and variant is instantiated in its own translation unit.
#pragma once

#include "pa_kernels.h"

namespace simpler_hip {
namespace pa {
namespace {

template <int BS, int D, typename OutT, typename ET, bool APPEND>
KernelPair gqa_pair() {
    // The fused append runs with one row tile per worker only: the host sends
    // shapes with more tiles per worker through a separate append launch.
    if constexpr (APPEND)
        return KernelPair{pa_decode_kernel<BS, D, D, OutT, 1, false, ET, true>, nullptr, false, D == 128};
    KernelPair k{pa_decode_kernel<BS, D, D, OutT, 1, false, ET, APPEND>,
                 pa_decode_kernel<BS, D, D, OutT, kMaxWavesPerWorker, false, ET, APPEND>, false, D == 128};
    if constexpr (D == 128) k.main_pair = pa_decode_kernel<BS, D, D, OutT, 1, false, ET, APPEND, 2>;
    return k;
}

// Block sizes 16..128 and head dims 16..256 (a block with more than 16384
// elements of K or V runs run_segment_big).
template <int BS, typename OutT, typename ET, bool APPEND>
KernelPair gqa_by_dim(int d) {
    switch (d) {
        case 16: return gqa_pair<BS, 16, OutT, ET, APPEND>();
        case 32: return gqa_pair<BS, 32, OutT, ET, APPEND>();
        case 64: return gqa_pair<BS, 64, OutT, ET, APPEND>();
        case 128: return gqa_pair<BS, 128, OutT, ET, APPEND>();
        case 256: return gqa_pair<BS, 256, OutT, ET, APPEND>();
        default: return KernelPair{};
    }
}

template <typename OutT, typename ET, bool APPEND>
KernelPair gqa_by_block(int bs, int d) {
    switch (bs) {
        case 16: return gqa_by_dim<16, OutT, ET, APPEND>(d);
        case 32: return gqa_by_dim<32, OutT, ET, APPEND>(d);
        case 64: return gqa_by_dim<64, OutT, ET, APPEND>(d);
        case 128: return gqa_by_dim<128, OutT, ET, APPEND>(d);
        default: return KernelPair{};
    }
}

}  // namespace
}  // namespace pa
}  // namespace simpler_hip
