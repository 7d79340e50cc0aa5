// Library-internal entry points of the decode (not exported).
#pragma once

#include <stddef.h>

#include "simpler_hip/pa_decode.h"

namespace simpler_hip {

// Enqueues a kernel that zeroes `bytes` bytes at device pointer `p` on
// `stream` (no memset node, so it may run under graph capture).
int zero_fill(void *p, size_t bytes, void *stream);

// simpler_hip_pa_decode with the merge kernel also storing the final error
// word into *err_mirror, host-visible pinned memory, so a caller that waits on
// the stream can read it without a device-to-host copy. Returns what
// simpler_hip_pa_decode returns; with batch 0 nothing is launched and
// *err_mirror is left as it is.
int pa_decode_with_mirror(const SimplerHipPaDecodeArgs *a, void *workspace, size_t workspace_bytes, void *stream,
                          unsigned *err_mirror);

}  // namespace simpler_hip
