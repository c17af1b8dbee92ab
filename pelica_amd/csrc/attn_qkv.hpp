// Launch parameters of the q/k/v step before attention (attn_qkv.hip).
#pragma once
#include "attn_common.hpp"

namespace pelica {

struct QkvParams {
    float* q;             // [token][n_head][hd] f32, rotated in place
    const float* k;       // [token][n_kv][hd] f32
    const float* v;
    int64_t tok_q, tok_kv;  // floats between consecutive tokens of q, of k / v
    const float* q_norm;  // [hd] or null
    const float* k_norm;
    float eps;
    const float* table;   // rope (cos, sin) rows, null = no rope
    int rot, neox, table_split;
    uint16_t* k_cache;
    uint16_t* v_cache;
    const int32_t* seq_len;
    const int64_t* seq_off;
    int64_t row_stride;   // f16 values between cache rows
    int kv_len, n_head, n_kv, hd, T, n_seq, ring_cap;
};

hipError_t launch_qkv(const QkvParams& p, hipStream_t st);

}  // namespace pelica
