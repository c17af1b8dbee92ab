// The step before attention, fused: per-head RMS norm of the q and k heads,
// rotary embedding of q and k, q written back, the new k and v rows rounded
// to f16 into the cache (linear or ring rows).  qk_dec
// (src/moe_kernels.rs:304-378) and ROPE_KV_T (src/oss_batch.rs:113-170);
// the f16 rows replace gpt-oss's f32 cache (src/oss.rs:615-616).
//
// One wave per (token, head slot): slots [0, n_head) are q heads, then n_kv
// k heads, then n_kv v heads; lane l holds elements l + 64 i of its head.
// The norm is a wave reduction; the rotation reads each element's partner
// through the wave's LDS row.  HBM-bound: every byte is touched once.
#include "attn_prof.hpp"
#include "attn_qkv.hpp"

namespace pelica {

template <int HD>
__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(QkvParams p) {
    constexpr int EPL = HD / 64;  // elements per lane
    __shared__ float row[4][HD];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int slot = blockIdx.x * 4 + wave;
    const int t = blockIdx.y, s = blockIdx.z;
    const int n_slot = p.n_head + 2 * p.n_kv;
    if (slot >= n_slot) return;
    const int kind = slot < p.n_head ? 0 : slot < p.n_head + p.n_kv ? 1 : 2;  // q, k, v
    const int h = kind == 0 ? slot : kind == 1 ? slot - p.n_head : slot - p.n_head - p.n_kv;
    const size_t tok = (size_t)s * p.T + t;
    const float* src = kind == 0 ? p.q + tok * p.tok_q + (size_t)h * HD
                     : (kind == 1 ? p.k : p.v) + tok * p.tok_kv + (size_t)h * HD;
    const int len = p.seq_len ? p.seq_len[s] : p.kv_len;
    if (len < p.T || len > p.kv_len) return;  // (attention skips such sequences too)
    const int pos = len - p.T + t;

    float x[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) x[i] = src[lane + 64 * i];

    const float* w = kind == 0 ? p.q_norm : kind == 1 ? p.k_norm : nullptr;
    if (w) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) ss += x[i] * x[i];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
        const float inv = 1.f / __builtin_sqrtf(ss / (float)HD + p.eps);
#pragma unroll
        for (int i = 0; i < EPL; ++i) x[i] = x[i] * inv * w[lane + 64 * i];
    }

    if (kind < 2 && p.table) {
        float* r = row[wave];
#pragma unroll
        for (int i = 0; i < EPL; ++i) r[lane + 64 * i] = x[i];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        const int half = p.rot / 2;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = lane + 64 * i;
            if (e >= p.rot) continue;
            int j, a, b;
            if (p.neox) {
                j = e < half ? e : e - half;
                a = j;
                b = j + half;
            } else {
                j = e >> 1;
                a = 2 * j;
                b = 2 * j + 1;
            }
            float cs, sn;
            if (p.table_split <= 0) {
                const float2 c = *reinterpret_cast<const float2*>(p.table + ((size_t)pos * half + j) * 2);
                cs = c.x;
                sn = c.y;
            } else {
                // angle addition of the rows for pos / 256 and pos % 256
                const float2 c1 = *reinterpret_cast<const float2*>(p.table + ((size_t)(pos >> 8) * half + j) * 2);
                const float2 c2 =
                    *reinterpret_cast<const float2*>(p.table + ((size_t)(p.table_split + (pos & 255)) * half + j) * 2);
                cs = c1.x * c2.x - c1.y * c2.y;
                sn = c1.y * c2.x + c1.x * c2.y;
            }
            const float x0 = r[a], x1 = r[b];
            x[i] = e == a ? x0 * cs - x1 * sn : x0 * sn + x1 * cs;
        }
    }

    if (kind == 0) {
        float* dst = p.q + tok * p.tok_q + (size_t)h * HD;
#pragma unroll
        for (int i = 0; i < EPL; ++i) dst[lane + 64 * i] = x[i];
    } else {
        const int64_t base = p.seq_off ? p.seq_off[s] : (int64_t)s * (p.ring_cap ? p.ring_cap : p.kv_len);
        const int64_t rowi = base + (p.ring_cap ? pos % p.ring_cap : pos);
        uint16_t* dst = (kind == 1 ? p.k_cache : p.v_cache) + rowi * p.row_stride + (int64_t)h * HD;
#pragma unroll
        for (int i = 0; i < EPL; ++i) dst[lane + 64 * i] = __builtin_bit_cast(uint16_t, (_Float16)x[i]);
    }
}

hipError_t launch_qkv(const QkvParams& p, hipStream_t st) {
    const int n_slot = p.n_head + 2 * p.n_kv;
    const dim3 grid((n_slot + 3) / 4, p.T, p.n_seq);
    ProfScope ps(kProfQkv, st);
    switch (p.hd) {
        case 64: hipLaunchKernelGGL(qkv_rope_cache_kernel<64>, grid, dim3(256), 0, st, p); break;
        case 128: hipLaunchKernelGGL(qkv_rope_cache_kernel<128>, grid, dim3(256), 0, st, p); break;
        case 256: hipLaunchKernelGGL(qkv_rope_cache_kernel<256>, grid, dim3(256), 0, st, p); break;
        default: return hipErrorNotSupported;
    }
    return hipGetLastError();
}

}  // namespace pelica
