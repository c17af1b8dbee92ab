// Launch parameters of the prefill kernel (attn_prefill.hip).
#pragma once
#include "attn_common.hpp"

namespace pelica {

struct PrefillParams {
    const void* q;       // f16, or f32 with f32
    const uint16_t* k;
    const uint16_t* v;
    const float* sinks;
    void* out;           // f16, or f32 with f32
    bool f32;            // f32 queries and output
    int64_t q_tok, o_tok;  // values between consecutive query / output tokens
    const int32_t* seq_len;
    const int64_t* seq_off;
    int64_t row_stride;  // f16 values between cache rows
    int kv_len, n_head, n_kv, hd, hpk, T, n_seq;
    int window, ring_cap;
    float qscale;  // scale * log2(e)
    // round mode (a prompt's keys in rounds): k, v hold the rows of key
    // positions [key_begin, key_end); state is the running (M natural-log,
    // L, O[hd]) per (token, head), read unless first; out may be null
    int key_begin, key_end, first;
    float* state;
};

// hipErrorNotSupported for shapes the kernel does not take
hipError_t launch_prefill(const PrefillParams& p, hipStream_t st);

}  // namespace pelica
