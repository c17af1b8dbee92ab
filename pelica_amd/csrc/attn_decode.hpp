// Launch parameters of the decode kernel (attn_decode.hip).
#pragma once
#include "attn_common.hpp"

namespace pelica {

// most key splits one query row may have (the combine stages one weight per
// split in LDS)
constexpr int kMaxSlots = 1024;
// Waves per decode workgroup (wg_heads kv heads x the rest waves each): 4,
// or 8 where two waves per SIMD fit the kernel's registers (head dim 64, up
// to 32 rows) and the call is large enough to want whole-row reads.
constexpr bool decode_can_use_8_waves(int hd, int rt) { return hd == 64 && rt <= 2; }

struct DecodeParams {
    // (field order: what the kernels read lies in the first 192 bytes, three
    // 64-byte kernel-argument lines; the first touch of a line is a memory
    // round trip, which costs ~0.5 us when it falls late in a kernel)
    const float* q;
    const uint16_t* k;
    const uint16_t* v;
    const float* sinks;
    float* out;
    float* ws_ml;      // [n_seq][n_kv][R][n_slot] x (max, sum), base-2 max
    float* ws_o;       // [n_seq][n_kv][R][n_slot][hd]
    const int32_t* seq_len;
    const int64_t* seq_off;
    int* ws_np;          // stream-K: pieces of each (sequence, row group x kv head) segment
    float* parts;        // non-null: write merge_dec partial slots here instead of out
    int64_t row_stride;  // f16 values between cache rows
    int64_t q_tok, o_tok;  // f32 values between consecutive query / output tokens
    int kr_lo, kr_hi;    // the call's key positions [kr_lo, kr_hi) (0, INT32_MAX: all);
                         // cache row 0 holds position kr_lo
    int kv_len, n_head, n_kv, hpk, T, R, n_seq, n_rg;
    int window, ring_cap;
    float qscale;        // scale * log2(e)
    int n_slot;          // key splits per (sequence, kv head, row group) in the grid
    int split_keys;      // keys per split, a multiple of 64
    int wg_heads;        // kv heads per workgroup: 4 (8-wave workgroups) or 1
    // stream-K over a ragged batch (no window, no ring; wg_heads 1): a 1-D
    // grid of sk_grid workgroups (0: a split grid) shares the batch's 64-key
    // blocks evenly, each at least sk_minb list positions; n_slot bounds the
    // pieces of a segment
    int sk_grid, sk_minb;
    int sk_restart;      // list positions charged at each segment's start (a piece's start-up cost)
    int rg_rows;         // query rows per row group (16 x row tiles)
    // read by the host-side launch code only
    int hd;
    bool sk;             // stream-K (sk_grid > 0)
    bool split_only;     // measurement: skip the combine (partials stay in the workspace)
};

hipError_t launch_decode(const DecodeParams& p, int rt, int nw, hipStream_t st);
// the in-order combine of the split partials in p.ws_ml / p.ws_o (hd 64, 128, 512)
hipError_t launch_combine(const DecodeParams& p, hipStream_t st);
// MLA: n_kv = 1, K = V = latent rows of 512, rows = tokens x heads (attn_mla.hip)
hipError_t launch_mla(const DecodeParams& p, hipStream_t st);
// zero n counters with a fill kernel (graph-capturable)
hipError_t launch_zero(unsigned* p, size_t n, hipStream_t st);

}  // namespace pelica
