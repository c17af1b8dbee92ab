// Merge of externally produced partial slots (the reference's merge_dec
// format: {M natural-log max, L, O[hd]} per slot, token and head) into the
// attention output, with optional sinks.
//
// Grid (n_head x dim slices, n_tokens): 512-thread workgroups per (token,
// head), as ATTN_M's grid (n_head, TMAX) (src/oss_batch.rs:395-425), each
// head's dims cut into slices when the grid would be small.  Thread (phase,
// dim pair) takes the slots c = phase (mod phases): all of a batch's loads
// (its (max, sum) pairs and its two dims of O) in flight at once, merged in
// slot order into a running (max, sum, O) state; then the phases' states
// are merged in phase order through LDS, the sink last (in the max and the
// denominator) — one memory round trip and one barrier per call, and the
// result does not depend on timing.  merge_dec_fast (src/moe_kernels.rs:
// 750-808) stages one weight per slot in workgroup memory instead; here the
// dim-pair threads of a phase each compute their slots' weights (16 exp2 a
// thread at 512 slots), which costs less than the staging's barriers.
#include "attn_common.hpp"
#include "attn_merge.hpp"
#include "attn_prof.hpp"

namespace pelica {

namespace {

constexpr int kThreads = 512;
constexpr int kBatch = 16;  // slots a thread loads at once (all in flight; 32 measured slower)

// (m, l, o) := (m, l, o) merged with (m2, l2, o2); m natural-log maxima
__device__ __forceinline__ void merge_ml(float& m, float& l, float2& o, float m2, float l2, float2 o2) {
    const float M = fmaxf(m, m2);
    const float ms = (M == -INFINITY) ? 0.f : M;
    const float a = fast_exp2((m - ms) * kLog2e), b = fast_exp2((m2 - ms) * kLog2e);
    l = l * a + l2 * b;
    o.x = o.x * a + o2.x * b;
    o.y = o.y * a + o2.y * b;
    m = M;
}

__global__ __launch_bounds__(kThreads) void partials_merge_kernel(int n_tok, int n_head, int hd, int dw, int n_parts,
                                                                  const float* __restrict__ parts,
                                                                  const float* __restrict__ sinks,
                                                                  float* __restrict__ out) {
    __shared__ float4 st_s[kThreads];  // each thread's merged state (m, l, o.x, o.y)
    const int nds = hd / dw;  // dim slices per head
    const int h = blockIdx.x / nds, d0 = dw * (blockIdx.x % nds), t = blockIdx.y, tid = threadIdx.x;
    const size_t stride = (size_t)n_tok * n_head * (hd + 2);  // floats between slots
    const float* ph = parts + ((size_t)t * n_head + h) * (hd + 2);
    const int dp_n = dw / 2;                   // dim pairs of the slice (dw <= 1024: <= 512)
    const int n_ph = kThreads / dp_n;          // slot phases
    const int ph_i = tid / dp_n, dp = tid % dp_n;
    const bool worker = ph_i < n_ph;
    const float* po = ph + 2 + d0 + 2 * dp;

    // this thread's slots c = ph_i + n_ph j, kBatch at a time: every load of
    // a batch in flight, then merged in slot order into the running state
    float m = -INFINITY, l = 0.f;
    float2 o = make_float2(0.f, 0.f);
    for (int c0 = ph_i; c0 < n_parts; c0 += n_ph * kBatch) {
        float2 ml[kBatch], ov[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int c = c0 + n_ph * j;
            const bool ld = worker && c < n_parts;
            ml[j] = ld ? *reinterpret_cast<const float2*>(ph + (size_t)c * stride) : make_float2(-INFINITY, 0.f);
            ov[j] = ld ? *reinterpret_cast<const float2*>(po + (size_t)c * stride) : make_float2(0.f, 0.f);
        }
        // the batch's max first: one rescale of the running state per batch
        float mb = m;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) mb = fmaxf(mb, ml[j].x);
        const float ms = (mb == -INFINITY) ? 0.f : mb;
        const float f = fast_exp2((m - ms) * kLog2e);
        l *= f;
        o.x *= f;
        o.y *= f;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const float w = fast_exp2((ml[j].x - ms) * kLog2e);
            l += ml[j].y * w;
            o.x += ov[j].x * w;
            o.y += ov[j].y * w;
        }
        m = mb;
    }
    // the phases' states, merged in phase order by the dim pair's thread
    st_s[tid] = make_float4(m, l, o.x, o.y);
    __syncthreads();
    if (tid < dp_n) {
        // two passes over the phases (their max, then their weighted sums
        // in phase order): independent exp2s instead of a chain of merges
        float M = -INFINITY;
        for (int q = 0; q < n_ph; ++q) M = fmaxf(M, st_s[q * dp_n + tid].x);
        const float ms = (M == -INFINITY) ? 0.f : M;
        float L = 0.f;
        float2 O = make_float2(0.f, 0.f);
        for (int q = 0; q < n_ph; ++q) {
            const float4 x = st_s[q * dp_n + tid];
            const float w = fast_exp2((x.x - ms) * kLog2e);
            L += x.y * w;
            O.x += x.z * w;
            O.y += x.w * w;
        }
        if (sinks) merge_ml(M, L, O, sinks[h], 1.f, make_float2(0.f, 0.f));  // sink: max and denominator
        const float inv = 1.f / L;
        *reinterpret_cast<float2*>(out + ((size_t)t * n_head + h) * hd + d0 + 2 * tid) = make_float2(O.x * inv, O.y * inv);
    }
}

}  // namespace

hipError_t launch_partials_merge(int n_tok, int n_head, int hd, int n_parts, const float* parts, const float* sinks,
                                 float* out, hipStream_t st) {
    if (hd <= 0 || hd % 2 || hd > 2 * kThreads) return hipErrorInvalidValue;
    // dim slices: halve the slice (down to 32 dims, even, dividing hd)
    // while the grid is below 256 workgroups (512 slots x 32 heads: one
    // token 9.1 -> 7.9 us with 32-dim slices, 11.0 with 16; four tokens
    // 13.2 -> 11.6 us with 64-dim slices)
    int dw = hd;
    while ((long long)n_head * n_tok * (hd / dw) < 256 && dw % 4 == 0 && dw / 2 >= 32) dw /= 2;
    ProfScope ps(kProfMerge, st);
    hipLaunchKernelGGL(partials_merge_kernel, dim3(n_head * (hd / dw), n_tok), dim3(kThreads), 0, st, n_tok, n_head, hd,
                       dw, n_parts, parts, sinks, out);
    return hipGetLastError();
}

}  // namespace pelica
