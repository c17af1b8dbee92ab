// Causal flash-attention prefill for gfx950: f16 Q/K/V, f32 softmax and
// accumulation, f16 output, learned sinks and sliding windows in the tile loop.
//
// Work split.  A workgroup (NW waves) owns one kv head of one sequence and a
// block of consecutive prompt tokens; its query rows are (token, head) pairs
// of that kv head's GQA group, so each K/V tile staged in LDS serves every
// head of the group.  Each wave holds RT tiles of 16 rows.  Keys stream in
// 64-key tiles, double-buffered in LDS (global loads of tile j+1 are in
// flight while tile j is computed).
//
// Per tile and wave:
//   S^T[key][row] = K Q^T  — v_mfma_f32_16x16x32_f16, K from LDS (ds_read_b128
//                            in the A-operand layout), Q resident in VGPRs;
//   softmax in base 2 with a lazy running max: the max moves (and O, l are
//   rescaled) only when some row's tile max exceeds it by more than 2^8, so
//   most tiles skip the rescale;  masking (causal, window) only on the tiles
//   that straddle a boundary;
//   O^T[dim][row] += V^T P^T — V read from LDS with ds_read_b64_tr_b16 into the
//   A operand, P (f16) as the B operand straight from the score registers.
// Sinks seed the running state (max = sink, sum = 1), as attn_p does
// (src/oss_prefill.rs:391-526); the window mask is j > pos || j + win <= pos
// (src/oss_prefill.rs:408).  Workgroups are ordered so that each XCD works on
// one kv head (its K/V stays in that XCD's L2) and the longest key ranges
// start first.
#include "attn_prefill.hpp"

namespace pelica {

template <int HD, int RT, int NW>
__global__ __launch_bounds__(64 * NW) void prefill_kernel(PrefillParams p, int n_tb, int TB) {
    constexpr int DS = HD / 32;
    constexpr int DT = HD / 16;
    constexpr int KP = HD + 8;                  // LDS row pitch (halfs)
    constexpr int PIECES = 64 * HD / 8;         // 16-byte pieces per 64-key tile
    constexpr int PPT = PIECES / (64 * NW);     // pieces per thread (K, and V)
    static_assert(PIECES % (64 * NW) == 0, "tile pieces must split evenly");
    __shared__ __attribute__((aligned(16))) _Float16 ks[2][64 * KP];
    __shared__ __attribute__((aligned(16))) _Float16 vs[2][64 * KP];

    // XCD-aware block order: dispatch goes round-robin over the 8 XCDs, so
    // give each XCD a contiguous range of logical blocks (same kv head)
    const int nblk = gridDim.x;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int tb = n_tb - 1 - bid % n_tb;  // longest key ranges first
    const int rest = bid / n_tb;
    const int kvh = rest % p.n_kv, s = rest / p.n_kv;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    const int len = p.seq_len ? p.seq_len[s] : p.kv_len;
    if (len < p.T || len <= 0) return;
    const int64_t row0 = p.seq_off ? p.seq_off[s] : (int64_t)s * (p.ring_cap ? p.ring_cap : p.kv_len);
    const int t0 = tb * TB;
    if (t0 >= p.T) return;
    const int t1 = min(t0 + TB, p.T);  // tokens [t0, t1)
    const int pos_first = len - p.T + t0, pos_last = len - p.T + t1 - 1;
    const int lo_first = (p.window > 0 && pos_first + 1 > p.window) ? pos_first + 1 - p.window : 0;
    const int lo_last = (p.window > 0 && pos_last + 1 > p.window) ? pos_last + 1 - p.window : 0;

    // this lane's rows: Q as B operand, position and window start
    half8 qb[RT][DS];
    int posr[RT], lor[RT];
    bool valid[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = (wave * RT + rt) * 16 + c16;
        const int t = t0 + r / p.hpk;
        valid[rt] = r < TB * p.hpk && t < t1;
        if (valid[rt]) {
            const int h = kvh * p.hpk + r % p.hpk;
            const uint16_t* qp = p.q + ((size_t)(s * p.T + t) * p.n_head + h) * HD + 8 * g;
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) qb[rt][ds] = load16(qp + 32 * ds);
            posr[rt] = len - p.T + t;
            lor[rt] = (p.window > 0 && posr[rt] + 1 > p.window) ? posr[rt] + 1 - p.window : 0;
        } else {
#pragma unroll
            for (int ds = 0; ds < DS; ++ds)
#pragma unroll
                for (int j = 0; j < 8; ++j) qb[rt][ds][j] = 0;
            posr[rt] = -1;
            lor[rt] = 0;
        }
    }

    // running state; a sink starts it at (max = sink, sum = 1)
    float m[RT], l[RT];
    float4v o[DT][RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m[rt] = -INFINITY;
        l[rt] = 0.f;
        if (p.sinks && valid[rt]) {
            const int r = (wave * RT + rt) * 16 + c16;
            m[rt] = p.sinks[kvh * p.hpk + r % p.hpk] * kLog2e;
            l[rt] = g == 0 ? 1.f : 0.f;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt][rt] = float4v{0.f, 0.f, 0.f, 0.f};
    }

    const uint16_t* kbase = p.k + (size_t)kvh * HD;
    const uint16_t* vbase = p.v + (size_t)kvh * HD;
    const int kb0 = lo_first & ~63;
    const int n_tiles = (pos_last - kb0) / 64 + 1;

    u32x4 kr[PPT], vr[PPT];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int piece = i * 64 * NW + tid;
            const int key = piece / (HD / 8), col = piece % (HD / 8);
            int j = min(kb + key, len - 1);
            const int64_t row = row0 + (p.ring_cap ? j % p.ring_cap : j);
            kr[i] = *reinterpret_cast<const u32x4*>(kbase + row * p.row_stride + 8 * col);
            vr[i] = *reinterpret_cast<const u32x4*>(vbase + row * p.row_stride + 8 * col);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int piece = i * 64 * NW + tid;
            const int key = piece / (HD / 8), col = piece % (HD / 8);
            *reinterpret_cast<u32x4*>(&ks[buf][key * KP + 8 * col]) = kr[i];
            *reinterpret_cast<u32x4*>(&vs[buf][key * KP + 8 * col]) = vr[i];
        }
    };

    load_tile(kb0);
    store_tile(0);
    __syncthreads();

    for (int it = 0; it < n_tiles; ++it) {
        const int kb = kb0 + 64 * it;
        const int buf = it & 1;
        const bool more = it + 1 < n_tiles;
        if (more) load_tile(kb + 64);

        const _Float16* kt_lds = ks[buf];
        const _Float16* vt_lds = vs[buf];

        // S^T = K Q^T
        float4v sc[4][RT];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            half8 ka[DS];
#pragma unroll
            for (int ds = 0; ds < DS; ++ds)
                ka[ds] = *reinterpret_cast<const half8*>(kt_lds + (16 * kt + c16) * KP + 32 * ds + 8 * g);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) acc = mfma16(ka[ds], qb[rt][ds], acc);
                sc[kt][rt] = acc;
            }
        }

        // boundary tiles: causal / window mask
        if (kb + 63 > pos_first || kb < lo_last) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kb + 16 * kt + 4 * g + i;
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        if (key < lor[rt] || key > posr[rt]) sc[kt][rt][i] = -INFINITY;
                }
        }

        // tile max per row (raw scores; the scale is positive)
        float bm[RT];
        bool grow = false;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float x = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) x = fmaxf(x, sc[kt][rt][i]);
            bm[rt] = group4_max(x) * p.qscale;
            grow |= bm[rt] > m[rt] + 8.f;
        }
        if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const float mn = fmaxf(m[rt], bm[rt]);
                if (mn != m[rt]) {
                    const float c = fast_exp2(m[rt] - mn);  // 0 when m was -inf
                    l[rt] *= c;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) o[dt][rt] *= c;
                    m[rt] = mn;
                }
            }
        }

        half8 pb[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float ms = (m[rt] == -INFINITY) ? 0.f : m[rt];
            float ls = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pe = fast_exp2(__builtin_fmaf(sc[kt][rt][i], p.qscale, -ms));
                    ls += pe;
                    pb[rt][kt >> 1][(kt & 1) * 4 + i] = (_Float16)pe;
                }
            l[rt] += ls;
        }

        // O^T += V^T P^T
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const _Float16* a = vt_lds + (32 * u + 4 * g + (c16 >> 2)) * KP + 16 * dt + 4 * (c16 & 3);
                const half8 va = cat8(lds_read_tr(a), lds_read_tr(a + 16 * KP));
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) o[dt][rt] = mfma16(va, pb[rt][u], o[dt][rt]);
            }

        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const float lt = group4_sum(l[rt]);
        if (!valid[rt]) continue;
        const int r = (wave * RT + rt) * 16 + c16;
        const int t = t0 + r / p.hpk, h = kvh * p.hpk + r % p.hpk;
        const float inv = 1.f / lt;
        uint16_t* op = p.out + ((size_t)(s * p.T + t) * p.n_head + h) * HD + 4 * g;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const half4 hv = {(_Float16)(o[dt][rt][0] * inv), (_Float16)(o[dt][rt][1] * inv),
                              (_Float16)(o[dt][rt][2] * inv), (_Float16)(o[dt][rt][3] * inv)};
            *reinterpret_cast<half4*>(op + 16 * dt) = hv;
        }
    }
}

template <int HD, int RT, int NW>
static hipError_t launch(const PrefillParams& p, hipStream_t st) {
    constexpr int ROWS = NW * RT * 16;
    if (p.hpk > ROWS) return hipErrorNotSupported;
    const int TB = ROWS / p.hpk;
    const int n_tb = (p.T + TB - 1) / TB;
    const long long nblk = (long long)n_tb * p.n_kv * p.n_seq;
    if (nblk > 0x7fffffff) return hipErrorNotSupported;
    hipLaunchKernelGGL((prefill_kernel<HD, RT, NW>), dim3((unsigned)nblk), dim3(64 * NW), 0, st, p, n_tb, TB);
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillParams& p, hipStream_t st) {
    if (p.hd == 64) return launch<64, 4, 4>(p, st);
    if (p.hd == 128) return launch<128, 2, 4>(p, st);
    return hipErrorNotSupported;
}

}  // namespace pelica
