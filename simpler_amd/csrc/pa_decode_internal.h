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

// The KV append (kv_cache.hip) for a decode's new tokens: the q_len new
// tokens of sequence b, rows [b, j] of key_new / value_new ([batch, q_len,
// num_kv_heads, head_dim] contiguous), go to positions context_lens[b] - q_len
// + j at the slots the block table gives. A position below 0 (a length below
// q_len) sets `bad_length` in *error_flag; positions past the table row and
// out-of-pool blocks are not written either (the decode reports both). `a`
// is validated by the caller.
int launch_paged_append(const SimplerHipPaDecodeArgs *a, const void *key_new, const void *value_new,
                        unsigned *error_flag, unsigned bad_length, void *stream);

// The decode prelude (kv_cache.hip) over the same tokens: the bf16 query rows
// into q_out ([batch, q_len, num_heads, head_dim]) and the new K/V rows into
// the caches, as simpler_hip_qk_norm_rope_append computes them; a position
// below 0 or past the RoPE table sets `bad_length` in *error_flag (its query
// row is zero and its cache rows are not written).
int launch_paged_prelude(const SimplerHipPaDecodeArgs *a, const SimplerHipDecodePreludeArgs *pre, void *q_out,
                         unsigned *error_flag, unsigned bad_length, void *stream);

}  // namespace simpler_hip
