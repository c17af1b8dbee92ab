// Merge of externally produced partial slots (the reference's merge_dec
// format: {M natural-log max, L, O[hd]} per slot, token and head) into the
// attention output, with optional sinks.
//
// Grid (n_head x dim slices, n_tokens): 512-thread workgroups per (token,
// head), as ATTN_M's grid (n_head, TMAX) (src/oss_batch.rs:395-425), each
// head's dims cut into slices when the grid would be small (every slice
// reduces the slots' (max, sum) pairs itself: 8 bytes a slot against its
// dw * 4 of O).  As merge_dec_fast
// does (src/moe_kernels.rs:750-808), each slot's weight e^(M_c - M) is
// computed once, by one thread, into LDS (tiles of kTile slots); then thread
// (phase, dim pair) sums its phase's slots c = phase (mod phases) with those
// weights, kBatch loads in flight at a time, and the phases are added in a
// fixed order through LDS — the result does not depend on timing.  The
// slots' (max, sum) pairs and the first O loads are requested together with
// the max pass, so the merge costs about one memory round trip per batch.
#include "attn_common.hpp"
#include "attn_merge.hpp"
#include "attn_prof.hpp"

namespace pelica {

namespace {

constexpr int kThreads = 512;
constexpr int kTile = 2048;   // slot (max, sum) pairs staged in LDS per pass
constexpr int kBatch = 32;    // O loads in flight per thread

__device__ __forceinline__ float block_reduce(float x, float* red, bool is_max) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float y = __shfl_xor(x, off, 64);
        x = is_max ? fmaxf(x, y) : x + y;
    }
    if (lane == 0) red[wave] = x;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(kThreads) void partials_merge_kernel(int n_tok, int n_head, int hd, int dw, int n_parts,
                                                                  const float* __restrict__ parts,
                                                                  const float* __restrict__ sinks,
                                                                  float* __restrict__ out) {
    __shared__ float2 ml_s[kTile];   // this tile's (max, sum) pairs, then (weight, -)
    __shared__ float red[kThreads / 64];
    __shared__ float2 acc_s[kThreads];
    const int nds = hd / dw;  // dim slices per head
    const int h = blockIdx.x / nds, d0 = dw * (blockIdx.x % nds), t = blockIdx.y, tid = threadIdx.x;
    const size_t stride = (size_t)n_tok * n_head * (hd + 2);  // floats between slots
    const float* ph = parts + ((size_t)t * n_head + h) * (hd + 2);
    const int dp_n = dw / 2;                   // dim pairs of the slice (dw <= 1024: <= 512)
    const int n_ph = kThreads / dp_n;          // slot phases
    const int ph_i = tid / dp_n, dp = tid % dp_n;
    const bool worker = ph_i < n_ph;
    const float* po = ph + 2 + d0 + 2 * dp;
    const float sk = sinks ? sinks[h] : -INFINITY;

    // the largest max (natural log) over every slot and the sink
    float M = sk;
    for (int c = tid; c < n_parts; c += kThreads) M = fmaxf(M, ph[c * stride]);

    float L = 0.f;
    float2 o = make_float2(0.f, 0.f);
    float2 v[kBatch];
    auto load_batch = [&](int t0, int n, int x0) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int x = x0 + n_ph * j;
            v[j] = worker && x < n ? *reinterpret_cast<const float2*>(po + (size_t)(t0 + x) * stride)
                                   : make_float2(0.f, 0.f);
        }
    };
    // the first tile's (max, sum) pairs into LDS and its first O batch into
    // registers, both in flight while the max is reduced
    int n = min(kTile, n_parts);
    for (int x = tid; x < n; x += kThreads) ml_s[x] = *reinterpret_cast<const float2*>(ph + (size_t)x * stride);
    load_batch(0, n, ph_i);
    M = block_reduce(M, red, true);  // (its barriers also publish ml_s)
    const float ms = (M == -INFINITY) ? 0.f : M;
    for (int t0 = 0; t0 < n_parts; t0 += kTile) {
        n = min(kTile, n_parts - t0);
        if (t0 > 0) {
            for (int x = tid; x < n; x += kThreads) ml_s[x] = *reinterpret_cast<const float2*>(ph + (size_t)(t0 + x) * stride);
            load_batch(t0, n, ph_i);
            __syncthreads();
        }
        // each slot's weight, once
        for (int x = tid; x < n; x += kThreads) {
            const float2 ml = ml_s[x];
            const float w = fast_exp2((ml.x - ms) * kLog2e);
            ml_s[x].x = w;
            L += ml.y * w;
        }
        __syncthreads();
        for (int x0 = ph_i; x0 < n; x0 += n_ph * kBatch) {
            if (x0 != ph_i) load_batch(t0, n, x0);
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int x = x0 + n_ph * j;
                const float w = worker && x < n ? ml_s[x].x : 0.f;
                o.x += v[j].x * w;
                o.y += v[j].y * w;
            }
        }
        __syncthreads();
    }
    L = block_reduce(L, red, false);
    if (sinks) L += fast_exp2((sk - ms) * kLog2e);
    // phases in order
    acc_s[tid] = o;
    __syncthreads();
    if (tid < dp_n) {
        float2 r = acc_s[tid];
        for (int q = 1; q < n_ph; ++q) {
            const float2 y = acc_s[q * dp_n + tid];
            r.x += y.x;
            r.y += y.y;
        }
        const float inv = 1.f / L;
        *reinterpret_cast<float2*>(out + ((size_t)t * n_head + h) * hd + d0 + 2 * tid) = make_float2(r.x * inv, r.y * inv);
    }
}

}  // namespace

hipError_t launch_partials_merge(int n_tok, int n_head, int hd, int n_parts, const float* parts, const float* sinks,
                                 float* out, hipStream_t st) {
    if (hd <= 0 || hd % 2 || hd > 2 * kThreads) return hipErrorInvalidValue;
    // dim slices: halve the slice (down to 32 dims, even, dividing hd) while
    // the grid is below 128 workgroups (one token of 32 heads: 11.2 -> 9.2
    // us; four tokens, already 128 workgroups: slicing further cost 6 %)
    int dw = hd;
    while ((long long)n_head * n_tok * (hd / dw) < 128 && dw % 4 == 0 && dw / 2 >= 32) dw /= 2;
    ProfScope ps(kProfMerge, st);
    hipLaunchKernelGGL(partials_merge_kernel, dim3(n_head * (hd / dw), n_tok), dim3(kThreads), 0, st, n_tok, n_head, hd,
                       dw, n_parts, parts, sinks, out);
    return hipGetLastError();
}

}  // namespace pelica
