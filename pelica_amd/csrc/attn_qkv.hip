// The step before attention, fused: per-head RMS norm of the q and k heads,
// rotary embedding of q and k, q written back, the new k and v rows rounded
// to f16 into the cache (linear or ring rows).  qk_dec
// (src/moe_kernels.rs:304-378) and ROPE_KV_T (src/oss_batch.rs:113-170);
// the f16 rows replace gpt-oss's f32 cache (src/oss.rs:615-616).
//
// Head slots [0, n_head) are q heads, then n_kv k heads, then n_kv v heads;
// a lane holds 4 consecutive elements of its slot (16-byte accesses), a wave
// 64/(hd/4) slots of a few consecutive tokens.  The norm is a reduction over the slot's lanes; the
// rotation reads each element's partner through the slot's LDS row.
// HBM-bound: every byte is touched once.
#include "attn_prof.hpp"
#include "attn_qkv.hpp"

namespace pelica {

// 4 consecutive floats: one 16-byte access (VEC), or four
template <bool VEC>
__device__ __forceinline__ float4v load4(const float* p) {
    if (VEC) return *reinterpret_cast<const float4v*>(p);
    return float4v{p[0], p[1], p[2], p[3]};
}
template <bool VEC>
__device__ __forceinline__ void store4(float* p, const float4v& x) {
    if (VEC) {
        *reinterpret_cast<float4v*>(p) = x;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = x[i];
    }
}

// One lane per 4 consecutive elements of a head: HD/4 lanes per head, 64/(HD/4)
// heads (slots) per wave, TPW tokens per wave.  VEC: 16-byte loads and
// stores (q/k/v rows and strides 16-byte aligned, cache rows 8-byte
// aligned).  Every token's loads (row, norm weights, rotation rows) are
// requested before any is used: a wave keeps TPW x 1 KB of its rows in
// flight, not 1 KB.
template <int HD, bool VEC, int TPW>
__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(QkvParams p) {
    constexpr int LPH = HD / 4;     // lanes per head
    constexpr int HPW = 64 / LPH;   // heads per wave
    __shared__ float row[4][TPW][HPW][HD];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane / LPH, hl = lane % LPH, e0 = 4 * hl;
    const int slot = (blockIdx.x * 4 + wave) * HPW + sub;
    const int tb = blockIdx.y * TPW, s = blockIdx.z;
    const int n_slot = p.n_head + 2 * p.n_kv;
    const int len = seq_keys(p.seq_len, s, p.kv_len);
    if (len < p.T || len > p.kv_len) return;  // (attention skips such sequences too)
    // lanes of slots past the end keep to the wave's lane exchanges with
    // harmless values and store nothing
    const bool live = slot < n_slot;
    const int kind = !live ? 2 : slot < p.n_head ? 0 : slot < p.n_head + p.n_kv ? 1 : 2;  // q, k, v
    const int h = !live ? 0 : kind == 0 ? slot : kind == 1 ? slot - p.n_head : slot - p.n_head - p.n_kv;
    const float* src0 = kind == 0 ? p.q + (size_t)h * HD : (kind == 1 ? p.k : p.v) + (size_t)h * HD;
    const int64_t tok_stride = kind == 0 ? p.tok_q : p.tok_kv;

    float4v x[TPW];
#pragma unroll
    for (int ti = 0; ti < TPW; ++ti) {
        const int t = tb + ti;
        x[ti] = live && t < p.T ? load4<VEC>(src0 + ((size_t)s * p.T + t) * tok_stride + e0)
                                : float4v{0.f, 0.f, 0.f, 0.f};
    }

    // the norm weights and the rotation's (cos, sin) of this lane's elements
    // are requested with the rows, not after them
    const float* w = kind == 0 ? p.q_norm : kind == 1 ? p.k_norm : nullptr;
    const float4v wv = w ? load4<false>(w + e0) : float4v{1.f, 1.f, 1.f, 1.f};
    const bool rot = kind < 2 && p.table && e0 < p.rot;
    float2 cssn[TPW][4];
    if (rot) {
        const int half = p.rot / 2;
#pragma unroll
        for (int ti = 0; ti < TPW; ++ti) {
            const int pos = len - p.T + min(tb + ti, p.T - 1);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = e0 + i;
                const int j = e >= p.rot ? 0 : p.neox ? (e < half ? e : e - half) : e >> 1;
                if (p.table_split <= 0) {
                    cssn[ti][i] = *reinterpret_cast<const float2*>(p.table + ((size_t)pos * half + j) * 2);
                } else {
                    // angle addition of the rows for pos / 256 and pos % 256
                    const float2 c1 =
                        *reinterpret_cast<const float2*>(p.table + ((size_t)(pos >> 8) * half + j) * 2);
                    const float2 c2 = *reinterpret_cast<const float2*>(
                        p.table + ((size_t)(p.table_split + (pos & 255)) * half + j) * 2);
                    cssn[ti][i] = make_float2(c1.x * c2.x - c1.y * c2.y, c1.y * c2.x + c1.x * c2.y);
                }
            }
        }
    }

#pragma unroll
    for (int ti = 0; ti < TPW; ++ti) {
        // per-head RMS norm: the sum of squares over the head's LPH lanes
        float ss = x[ti][0] * x[ti][0] + x[ti][1] * x[ti][1] + x[ti][2] * x[ti][2] + x[ti][3] * x[ti][3];
#pragma unroll
        for (int off = LPH / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
        if (w) {
            const float inv = 1.f / __builtin_sqrtf(ss / (float)HD + p.eps);
#pragma unroll
            for (int i = 0; i < 4; ++i) x[ti][i] = x[ti][i] * inv * wv[i];
        }
        // rotary: element e of the first rot pairs with its partner (e +-
        // rot/2, or e ^ 1 for interleaved pairs), read through the head's
        // LDS row
        if (p.table && e0 < p.rot) *reinterpret_cast<float4v*>(row[wave][ti][sub] + e0) = x[ti];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    if (rot) {
        const int half = p.rot / 2;
#pragma unroll
        for (int ti = 0; ti < TPW; ++ti) {
            const float* r = row[wave][ti][sub];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = e0 + i;
                if (e >= p.rot) continue;
                int a, b;
                if (p.neox) {
                    a = e < half ? e : e - half;
                    b = a + half;
                } else {
                    a = e & ~1;
                    b = a + 1;
                }
                const float x0 = r[a], x1 = r[b];
                x[ti][i] = e == a ? x0 * cssn[ti][i].x - x1 * cssn[ti][i].y : x0 * cssn[ti][i].y + x1 * cssn[ti][i].x;
            }
        }
    }
    if (!live) return;

#pragma unroll
    for (int ti = 0; ti < TPW; ++ti) {
        const int t = tb + ti;
        if (t >= p.T) break;
        const size_t tok = (size_t)s * p.T + t;
        if (kind == 0) {
            store4<VEC>(p.q + tok * p.tok_q + (size_t)h * HD + e0, x[ti]);
        } else {
            const int pos = len - p.T + t;
            const int64_t base = p.seq_off ? p.seq_off[s] : (int64_t)s * (p.ring_cap ? p.ring_cap : p.kv_len);
            const int64_t rowi = base + (p.ring_cap ? pos % p.ring_cap : pos);
            uint16_t* dst = (kind == 1 ? p.k_cache : p.v_cache) + rowi * p.row_stride + (int64_t)h * HD + e0;
            uint16_t hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) hv[i] = __builtin_bit_cast(uint16_t, (_Float16)x[ti][i]);
            if (VEC) {
                *reinterpret_cast<u32x2*>(dst) = u32x2{hv[0] | (uint32_t)hv[1] << 16, hv[2] | (uint32_t)hv[3] << 16};
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[i] = hv[i];
            }
        }
    }
}

// tokens per wave (gpt-oss 4096-token step: 1 token 34.7 us, 2 30.3, 3 30.3,
// 4 30.0-30.8, 5 32.7, 6 33-35, 8 36.5)
constexpr int kQkvTpw = 4;

template <int HD>
static void launch_hd(const QkvParams& p, bool vec, dim3 grid, hipStream_t st) {
    if (vec) hipLaunchKernelGGL((qkv_rope_cache_kernel<HD, true, kQkvTpw>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((qkv_rope_cache_kernel<HD, false, kQkvTpw>), grid, dim3(256), 0, st, p);
}

hipError_t launch_qkv(const QkvParams& p, hipStream_t st) {
    const int n_slot = p.n_head + 2 * p.n_kv;
    const int hpw = 64 / (p.hd / 4);  // heads per wave
    const dim3 grid((n_slot + 4 * hpw - 1) / (4 * hpw), (p.T + kQkvTpw - 1) / kQkvTpw, p.n_seq);
    auto al = [](const void* q, int a) { return (reinterpret_cast<uintptr_t>(q) % a) == 0; };
    const bool vec = al(p.q, 16) && al(p.k, 16) && al(p.v, 16) && p.tok_q % 4 == 0 && p.tok_kv % 4 == 0 &&
                     al(p.k_cache, 8) && al(p.v_cache, 8) && p.row_stride % 4 == 0;
    ProfScope ps(kProfQkv, st);
    switch (p.hd) {
        case 64: launch_hd<64>(p, vec, grid, st); break;
        case 128: launch_hd<128>(p, vec, grid, st); break;
        case 256: launch_hd<256>(p, vec, grid, st); break;
        default: return hipErrorNotSupported;
    }
    return hipGetLastError();
}

}  // namespace pelica
