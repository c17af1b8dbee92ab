// Merge of merge_dec-format partial slots (attn_merge.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace pelica {

// parts[c][t][h][hd + 2] (c < n_parts, t < n_tok, h < n_head) -> out[t][h][hd];
// hd even, <= 1024
hipError_t launch_partials_merge(int n_tok, int n_head, int hd, int n_parts, const float* parts, const float* sinks,
                                 float* out, hipStream_t st);

}  // namespace pelica
