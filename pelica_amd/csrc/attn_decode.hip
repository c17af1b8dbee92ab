// Split-K flash-decode for gfx950: f32 queries, f16 KV cache, f32 output.
//
// Work split.  A workgroup is one wave (64 lanes) and owns (sequence s, kv
// head g, row group, key split).  All query rows that share kv head g — the
// GQA group times the pass's tokens (drafts) — ride in the same wave, so
// every K/V byte is read from HBM once.  Rows sit in the MFMA's 16-wide n
// dimension; keys stream through in blocks of 64.
//
// Per 64-key block:
//   K  global -> registers with 128-bit loads, already in the A-operand
//      layout of v_mfma_f32_16x16x32_f16 (lane: key l%16, 8 dims), so K
//      never touches LDS;
//   S^T[key][row] = K Q^T on MFMA.  Q is split into f16 hi + lo parts (two
//      MFMAs) so the scores keep ~fp32 accuracy;
//   online softmax in base 2 (log2(e) folded into the query scale), block
//      max and sums over the four 16-lane groups with permlane swaps;
//   V  global -> registers -> LDS (128-bit, row-major), read back with the
//      transposing ds_read_b64_tr_b16 into the A operand of O^T = V^T P^T;
//      P (f32) is split into f16 hi + lo as the B operand, straight from the
//      score registers (its key order matches the A operand's).
// Each split writes (max, sum, O[hd]) per row to the workspace; a combine
// kernel merges the splits in key order with the head's sink.  A single
// split writes the normalised output itself.
//
// Reference semantics: src/moe_kernels.rs:482-617 (attn_dec, merge_dec),
// src/oss_batch.rs:172-251 (ATTN_T: window, ring, sink), :253-425 (attn_s +
// ATTN_M: split partials, sink in max and denominator).
#include "attn_decode.hpp"

namespace pelica {

template <int HD, int RT>
__global__ __launch_bounds__(64) void decode_split_kernel(DecodeParams p) {
    constexpr int DS = HD / 32;  // 32-dim k-steps of the QK^T MFMA
    constexpr int DT = HD / 16;  // 16-dim output tiles
    constexpr int VP = HD + 8;   // LDS row pitch in halfs (breaks bank aliasing)
    constexpr int VPL = HD / 8;  // 16-byte V pieces per lane per block
    __shared__ __attribute__((aligned(16))) _Float16 vl[64 * VP];

    const int lane = threadIdx.x, g = lane >> 4, c16 = lane & 15;
    const int kvh = blockIdx.y % p.n_kv, rg = blockIdx.y / p.n_kv;
    const int s = blockIdx.z;
    const int len = p.seq_len ? p.seq_len[s] : p.kv_len;
    if (len < p.T || len <= 0) return;
    const int64_t row0 = p.seq_off ? p.seq_off[s] : (int64_t)s * (p.ring_cap ? p.ring_cap : p.kv_len);
    const int pos_first = len - p.T;
    const int lo_min = (p.window > 0 && pos_first + 1 > p.window) ? pos_first + 1 - p.window : 0;
    const int split0 = lo_min / p.split_keys;
    const int slot = blockIdx.x;
    const int kbeg = (split0 + slot) * p.split_keys;
    const int kend = min(kbeg + p.split_keys, len);
    if (kbeg >= kend) return;

    // queries of this lane's rows: hi/lo f16 pairs, scaled into base 2
    half8 qh[RT][DS], ql[RT][DS];
    int posr[RT], lor[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = rg * 16 * RT + 16 * rt + c16;
        if (r < p.R) {
            const int t = r / p.hpk, h = kvh * p.hpk + r % p.hpk;
            const float* qp = p.q + ((size_t)(s * p.T + t) * p.n_head + h) * HD + 8 * g;
            posr[rt] = pos_first + t;
            lor[rt] = (p.window > 0 && posr[rt] + 1 > p.window) ? posr[rt] + 1 - p.window : 0;
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const float4v a = *reinterpret_cast<const float4v*>(qp + 32 * ds);
                const float4v b = *reinterpret_cast<const float4v*>(qp + 32 * ds + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    _Float16 hi, lo;
                    split_f16(a[j] * p.qscale, hi, lo);
                    qh[rt][ds][j] = hi; ql[rt][ds][j] = lo;
                    split_f16(b[j] * p.qscale, hi, lo);
                    qh[rt][ds][4 + j] = hi; ql[rt][ds][4 + j] = lo;
                }
            }
        } else {
            posr[rt] = -1;
            lor[rt] = 0;
#pragma unroll
            for (int ds = 0; ds < DS; ++ds)
#pragma unroll
                for (int j = 0; j < 8; ++j) { qh[rt][ds][j] = 0; ql[rt][ds][j] = 0; }
        }
    }

    float m[RT], l[RT];
    float4v o[DT][RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m[rt] = -INFINITY;
        l[rt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt][rt] = float4v{0.f, 0.f, 0.f, 0.f};
    }

    const uint16_t* kbase = p.k + (size_t)kvh * HD;
    const uint16_t* vbase = p.v + (size_t)kvh * HD;
    auto row_of = [&](int key) -> int64_t {
        key = min(key, kend - 1);
        return row0 + (p.ring_cap ? key % p.ring_cap : key);
    };

    int kb = kbeg;
    if (lo_min > kbeg) kb = kbeg + ((lo_min - kbeg) & ~63);
    for (; kb < kend; kb += 64) {
        half8 kr[4][DS];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            const uint16_t* kp = kbase + row_of(kb + 16 * kt + c16) * p.row_stride + 8 * g;
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) kr[kt][ds] = load16(kp + 32 * ds);
        }
        u32x4 vr[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int piece = i * 64 + lane;
            const int key = piece / (HD / 8), col = piece % (HD / 8);
            vr[i] = *reinterpret_cast<const u32x4*>(vbase + row_of(kb + key) * p.row_stride + 8 * col);
        }

        // S^T = K Q^T (4 key tiles x RT row tiles), hi + lo queries
        float4v sc[4][RT];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    acc = mfma16(kr[kt][ds], qh[rt][ds], acc);
                    acc = mfma16(kr[kt][ds], ql[rt][ds], acc);
                }
                sc[kt][rt] = acc;
            }

        // V block into LDS (the previous block's reads are complete)
        __syncthreads();
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int piece = i * 64 + lane;
            const int key = piece / (HD / 8), col = piece % (HD / 8);
            *reinterpret_cast<u32x4*>(&vl[key * VP + 8 * col]) = vr[i];
        }

        // mask: row r sees keys [lor, posr]
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kb + 16 * kt + 4 * g + i;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    if (key < lor[rt] || key > posr[rt]) sc[kt][rt][i] = -INFINITY;
            }

        // online softmax, base 2
        half8 ph[RT][2], pl[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float bm = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) bm = fmaxf(bm, sc[kt][rt][i]);
            bm = group4_max(bm);
            const float mn = fmaxf(m[rt], bm);
            const float ms = (mn == -INFINITY) ? 0.f : mn;
            const float c = fast_exp2(m[rt] - ms);
            m[rt] = mn;
            float ls = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pe = fast_exp2(sc[kt][rt][i] - ms);
                    ls += pe;
                    _Float16 hi, lo;
                    split_f16(pe, hi, lo);
                    ph[rt][kt >> 1][(kt & 1) * 4 + i] = hi;
                    pl[rt][kt >> 1][(kt & 1) * 4 + i] = lo;
                }
            l[rt] = l[rt] * c + ls;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt][rt] *= c;
        }

        __syncthreads();
        // O^T += V^T P^T
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const _Float16* a = vl + (32 * u + 4 * g + (c16 >> 2)) * VP + 16 * dt + 4 * (c16 & 3);
                const half8 va = cat8(lds_read_tr(a), lds_read_tr(a + 16 * VP));
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    o[dt][rt] = mfma16(va, ph[rt][u], o[dt][rt]);
                    o[dt][rt] = mfma16(va, pl[rt][u], o[dt][rt]);
                }
            }
    }

#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const float lt = group4_sum(l[rt]);
        const int r = rg * 16 * RT + 16 * rt + c16;
        if (r >= p.R) continue;
        if (p.n_slot == 1) {
            // one split: normalise here, sink in max and denominator
            const int t = r / p.hpk, h = kvh * p.hpk + r % p.hpk;
            float w = 1.f, L = lt;
            if (p.sinks) {
                const float sk = p.sinks[h] * kLog2e;
                const float M = fmaxf(m[rt], sk);
                w = fast_exp2(m[rt] - M);
                L = lt * w + fast_exp2(sk - M);
            }
            const float f = w / L;
            float* op = p.out + ((size_t)(s * p.T + t) * p.n_head + h) * HD + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                *reinterpret_cast<float4v*>(op + 16 * dt) = o[dt][rt] * f;
        } else {
            const size_t idx = ((size_t)(s * p.n_kv + kvh) * p.R + r) * p.n_slot + slot;
            if (g == 0) {
                p.ws_ml[2 * idx] = m[rt];
                p.ws_ml[2 * idx + 1] = lt;
            }
            float* op = p.ws_o + idx * HD + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<float4v*>(op + 16 * dt) = o[dt][rt];
        }
    }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

// Combine of one row's split partials in key order, with the sink
// (src/moe_kernels.rs:585-617 merge_dec, src/oss_batch.rs:395-425 ATTN_M).
// Grid (n_kv * R, n_seq), 64 lanes.
template <int HD>
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeParams p) {
    __shared__ float w[kMaxSlots];
    const int lane = threadIdx.x;
    const int kvh = blockIdx.x / p.R, r = blockIdx.x % p.R;
    const int s = blockIdx.y;
    const int len = p.seq_len ? p.seq_len[s] : p.kv_len;
    if (len < p.T || len <= 0) return;
    const int t = r / p.hpk, h = kvh * p.hpk + r % p.hpk;
    const int pos_first = len - p.T;
    const int lo_min = (p.window > 0 && pos_first + 1 > p.window) ? pos_first + 1 - p.window : 0;
    const int split0 = lo_min / p.split_keys;
    const int pos = pos_first + t;
    const int lo = (p.window > 0 && pos + 1 > p.window) ? pos + 1 - p.window : 0;
    const int c0 = lo / p.split_keys - split0, c1 = pos / p.split_keys - split0;
    const size_t base = ((size_t)(s * p.n_kv + kvh) * p.R + r) * p.n_slot;

    const float sk = p.sinks ? p.sinks[h] * kLog2e : -INFINITY;
    float M = sk;
    for (int c = c0 + lane; c <= c1; c += 64) M = fmaxf(M, p.ws_ml[2 * (base + c)]);
    M = wave_max(M);
    const float ms = (M == -INFINITY) ? 0.f : M;
    float L = 0.f;
    for (int c = c0 + lane; c <= c1; c += 64) {
        const float wc = fast_exp2(p.ws_ml[2 * (base + c)] - ms);
        w[c - c0] = wc;
        L += p.ws_ml[2 * (base + c) + 1] * wc;
    }
    L = wave_sum(L);
    if (p.sinks) L += fast_exp2(sk - ms);
    __syncthreads();
    const float inv = 1.f / L;
    float* op = p.out + ((size_t)(s * p.T + t) * p.n_head + h) * HD;
    for (int d = lane; d < HD; d += 64) {
        float acc = 0.f;
        for (int c = c0; c <= c1; ++c) acc += p.ws_o[(base + c) * HD + d] * w[c - c0];
        op[d] = acc * inv;
    }
}

template <int HD, int RT>
static hipError_t launch_split(const DecodeParams& p, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((decode_split_kernel<HD, RT>), grid, dim3(64), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_decode(const DecodeParams& p, int rt, int n_rg, hipStream_t st) {
    dim3 grid(p.n_slot, p.n_kv * n_rg, p.n_seq);
    hipError_t e = hipErrorInvalidValue;
    if (p.hd == 64) {
        if (rt == 1) e = launch_split<64, 1>(p, grid, st);
        else if (rt == 2) e = launch_split<64, 2>(p, grid, st);
        else if (rt == 4) e = launch_split<64, 4>(p, grid, st);
    } else if (p.hd == 128) {
        if (rt == 1) e = launch_split<128, 1>(p, grid, st);
        else if (rt == 2) e = launch_split<128, 2>(p, grid, st);
    }
    if (e != hipSuccess || p.n_slot == 1) return e;
    dim3 cgrid(p.n_kv * p.R, p.n_seq);
    if (p.hd == 64) hipLaunchKernelGGL((decode_combine_kernel<64>), cgrid, dim3(64), 0, st, p);
    else hipLaunchKernelGGL((decode_combine_kernel<128>), cgrid, dim3(64), 0, st, p);
    return hipGetLastError();
}

}  // namespace pelica
