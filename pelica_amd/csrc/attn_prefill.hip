// Causal flash-attention prefill for gfx950: f16 Q/K/V, f32 softmax and
// accumulation, f16 output, learned sinks and sliding windows in the tile loop.
//
// Work split.  A workgroup (NW waves) owns one kv head of one sequence and a
// block of consecutive prompt tokens; its query rows are (token, head) pairs
// of that kv head's GQA group, so each K/V tile staged in LDS serves every
// head of the group.  Each wave holds RT tiles of 32 rows.  Keys stream in
// 64-key tiles, double-buffered in LDS: the next tile's global loads are in
// flight while the current one is computed.
//
// Per tile and wave, on v_mfma_f32_32x32x16_f16:
//   S^T[key][row] = K Q^T — K read from LDS (ds_read_b128, XOR-swizzled rows)
//     in the A-operand layout, Q resident in VGPRs as the B operand.  A lane
//     then holds 32 scores of ONE query row (column l%32), so the row max is
//     an in-lane max plus one permlane32 swap;
//   softmax in base 2 with a lazy running max: the max moves (and O, l are
//     rescaled) only when some row's tile max exceeds it by more than 2^8;
//     masking (causal, window) only on the tiles that straddle a boundary;
//   O^T[dim][row] += V^T P^T — V read from LDS with ds_read_b64_tr_b16 into
//     the A operand; P (f16) is the B operand straight from the score
//     registers: 8 consecutive accumulator elements are one operand.
// Sinks seed the running state (max = sink, sum = 1), as attn_p does
// (src/oss_prefill.rs:391-526); the window mask is j > pos || j + win <= pos
// (src/oss_prefill.rs:408).  Workgroups are ordered so that each XCD works on
// one kv head (its K/V stays in that XCD's L2) and the longest key ranges
// start first.
#include "attn_prefill.hpp"
#include "attn_prof.hpp"

namespace pelica {

typedef float float16v __attribute__((ext_vector_type(16)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));

// word 3 of a gfx9 buffer resource: 32-bit data format, raw addressing
constexpr int kBufferFlags = 0x00020000;

__device__ __forceinline__ float16v mfma32(const half8& a, const half8& b, const float16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// max / sum with the lane 32 apart
__device__ __forceinline__ float half_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float half_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// LDS byte offset of 16-byte piece p of key row k in a K tile: 16-byte pieces
// XOR-swizzled by the key so the A-operand reads (32 consecutive keys, one
// piece each) spread over all banks.
template <int HD>
__device__ __forceinline__ int k_slot(int k, int p) {
    return k * (HD * 2) + ((p ^ (k & 7)) << 4);
}

// ... and in a V tile: swizzled so the transposed reads of 4 consecutive
// keys at 16 dims hit distinct banks.
template <int HD>
__device__ __forceinline__ int v_slot(int k, int p) {
    return k * (HD * 2) + ((p ^ ((k & 3) << 1)) << 4);
}

template <int HD, int RT, int NW, bool RING>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(
    PrefillParams p, int n_tb, int TB) {
    constexpr int KS = HD / 16;                 // 16-dim k-steps of QK^T
    constexpr int DT = HD / 32;                 // 32-dim output tiles
    constexpr int TILE = 64 * HD * 2;           // bytes of a K (or V) tile
    constexpr int PPR = HD / 8;                 // 16-byte pieces per key row
    constexpr int PPT = 64 * PPR / (64 * NW);   // pieces per thread (K, and V)
    static_assert((64 * PPR) % (64 * NW) == 0, "tile pieces must split evenly");
    __shared__ __attribute__((aligned(16))) char lds[4 * TILE];  // K0 V0 K1 V1

    // XCD-aware block order: dispatch goes round-robin over the 8 XCDs, so
    // give each XCD a contiguous range of logical blocks (same kv head)
    const int nblk = gridDim.x;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int tb = n_tb - 1 - bid % n_tb;  // longest key ranges first
    const int rest = bid / n_tb;
    const int kvh = rest % p.n_kv, s = rest / p.n_kv;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h2 = lane >> 5, c32 = lane & 31;
    const int len = p.seq_len ? p.seq_len[s] : p.kv_len;
    if (len < p.T || len <= 0) return;
    const int64_t row0 = p.seq_off ? p.seq_off[s] : (int64_t)s * (p.ring_cap ? p.ring_cap : p.kv_len);
    const int t0 = tb * TB;
    if (t0 >= p.T) return;
    const int t1 = min(t0 + TB, p.T);  // tokens [t0, t1)
    const int pos_first = len - p.T + t0, pos_last = len - p.T + t1 - 1;
    const int lo_first = (p.window > 0 && pos_first + 1 > p.window) ? pos_first + 1 - p.window : 0;
    const int lo_last = (p.window > 0 && pos_last + 1 > p.window) ? pos_last + 1 - p.window : 0;

    // K/V tile loads through buffer resources over this sequence's rows of kv
    // head kvh: 32-bit offsets; rows past the sequence read as 0 (masked)
    const uint32_t stride_b = (uint32_t)p.row_stride * 2;
    const uint32_t nrec = (RING ? (uint32_t)p.ring_cap : (uint32_t)len) * stride_b;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.k + row0 * p.row_stride + (size_t)kvh * HD), (short)0, (int)nrec, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.v + row0 * p.row_stride + (size_t)kvh * HD), (short)0, (int)nrec, kBufferFlags);
    const int kb0 = lo_first & ~63;
    const int n_tiles = (pos_last - kb0) / 64 + 1;
    // thread piece i*64*NW + tid of a tile -> (key, 16-byte column)
    constexpr int KPI = 64 * NW / PPR;  // keys per piece round
    const int pkey = tid / PPR, pcol = tid % PPR;
    u32x4 kr[PPT], vr[PPT];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int key = KPI * i + pkey;
            const uint32_t off = RING ? ((kb + key) % p.ring_cap) * stride_b + 16 * pcol
                                      : (uint32_t)(kb + key) * stride_b + 16 * pcol;
            kr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
            vr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
        }
    };
    auto store_tile = [&](int buf) {
        char* kt = lds + buf * 2 * TILE;
        char* vt = kt + TILE;
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int key = KPI * i + pkey;
            *reinterpret_cast<u32x4*>(kt + k_slot<HD>(key, pcol)) = kr[i];
            *reinterpret_cast<u32x4*>(vt + v_slot<HD>(key, pcol)) = vr[i];
        }
    };
    load_tile(kb0);

    // this lane's query rows (column c32 of each 32-row tile): Q as the B
    // operand, position and window start
    half8 qb[RT][KS];
    int posr[RT], lor[RT];
    bool valid[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = (wave * RT + rt) * 32 + c32;
        const int t = t0 + r / p.hpk;
        valid[rt] = r < TB * p.hpk && t < t1;
        const int h = kvh * p.hpk + r % p.hpk;
        const uint16_t* qp = p.q + ((size_t)(s * p.T + (valid[rt] ? t : t0)) * p.n_head + (valid[rt] ? h : 0)) * HD + 8 * h2;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            qb[rt][ks] = load16(qp + 16 * ks);
            if (!valid[rt]) qb[rt][ks] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        posr[rt] = valid[rt] ? len - p.T + t : -1;
        lor[rt] = (p.window > 0 && posr[rt] + 1 > p.window) ? posr[rt] + 1 - p.window : 0;
    }

    // running state; a sink starts it at (max = sink, sum = 1)
    float m[RT], l[RT];
    float16v o[DT][RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m[rt] = -INFINITY;
        l[rt] = 0.f;
        if (p.sinks && valid[rt]) {
            const int r = (wave * RT + rt) * 32 + c32;
            m[rt] = p.sinks[kvh * p.hpk + r % p.hpk] * kLog2e;
            l[rt] = h2 == 0 ? 1.f : 0.f;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt][rt] = float16v{};
    }

    store_tile(0);
    __syncthreads();

    for (int it = 0; it < n_tiles; ++it) {
        const int kb = kb0 + 64 * it;
        const int buf = it & 1;
        const bool more = it + 1 < n_tiles;
        if (more) load_tile(kb + 64);
        const char* kt_lds = lds + buf * 2 * TILE;
        const char* vt_lds = kt_lds + TILE;

        // S^T = K Q^T: 2 key tiles x RT row tiles, k-steps outermost
        float16v sc[2][RT];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) sc[kt][rt] = float16v{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            half8 ka[2];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                ka[kt] = *reinterpret_cast<const half8*>(kt_lds + k_slot<HD>(32 * kt + c32, 2 * ks + h2));
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) sc[kt][rt] = mfma32(ka[kt], qb[rt][ks], sc[kt][rt]);
        }

        // boundary tiles only: causal / window mask.  Element i of key tile
        // kt is key kb + 32 kt + 8 (i / 4) + 4 h2 + i % 4.
        if (kb + 63 > pos_first || kb < lo_last) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = kb + 32 * kt + 8 * (i / 4) + 4 * h2 + (i % 4);
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
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i) x = fmaxf(x, sc[kt][rt][i]);
            bm[rt] = half_max(x) * p.qscale;
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

        // P = 2^(s*scale - m) as f16 B operands; chunk u (16 keys) is
        // elements 8(u%2) .. +7 of key tile u/2
        // (the row sum takes the f16 P the PV product uses, two at a time)
        half8 pb[4][RT];
        const half2 one2 = {(_Float16)1.f, (_Float16)1.f};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float ms = (m[rt] == -INFINITY) ? 0.f : m[rt];
            float ls = 0.f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    pb[u][rt][j] = (_Float16)fast_exp2(__builtin_fmaf(sc[u >> 1][rt][8 * (u & 1) + j], p.qscale, -ms));
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    ls = __builtin_amdgcn_fdot2(half2{pb[u][rt][2 * j], pb[u][rt][2 * j + 1]}, one2, ls, false);
            }
            l[rt] += ls;
        }

        // O^T += V^T P^T
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            half8 va[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                // lanes of 16-lane group G read keys 16u + 4 h2 + r (+8) at
                // dims 32 dt + 16 (G & 1) + 4 q; lane 4r + q of the group
                const int G = lane >> 4, r4 = (lane & 15) >> 2, q4 = lane & 3;
                const int key = 16 * u + 4 * h2 + r4, dim = 32 * dt + 16 * (G & 1) + 4 * q4;
                const _Float16* a0 = reinterpret_cast<const _Float16*>(vt_lds + v_slot<HD>(key, dim >> 3) + ((dim & 7) << 1));
                const _Float16* a1 = reinterpret_cast<const _Float16*>(vt_lds + v_slot<HD>(key + 8, dim >> 3) + ((dim & 7) << 1));
                va[dt] = cat8(lds_read_tr(a0), lds_read_tr(a1));
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) o[dt][rt] = mfma32(va[dt], pb[u][rt], o[dt][rt]);
        }

        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

    // O^T lane layout: dim 32 dt + 8 (i / 4) + 4 h2 + i % 4 of row c32
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const float lt = half_sum(l[rt]);
        if (!valid[rt]) continue;
        const int r = (wave * RT + rt) * 32 + c32;
        const int t = t0 + r / p.hpk, h = kvh * p.hpk + r % p.hpk;
        const float inv = 1.f / lt;
        uint16_t* op = p.out + ((size_t)(s * p.T + t) * p.n_head + h) * HD + 4 * h2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const half4 hv = {(_Float16)(o[dt][rt][4 * i4] * inv), (_Float16)(o[dt][rt][4 * i4 + 1] * inv),
                                  (_Float16)(o[dt][rt][4 * i4 + 2] * inv), (_Float16)(o[dt][rt][4 * i4 + 3] * inv)};
                *reinterpret_cast<half4*>(op + 32 * dt + 8 * i4) = hv;
            }
    }
}

template <int HD, int RT, int NW>
static hipError_t launch(const PrefillParams& p, hipStream_t st) {
    constexpr int ROWS = NW * RT * 32;
    if (p.hpk > ROWS) return hipErrorNotSupported;
    const int TB = ROWS / p.hpk;
    const int n_tb = (p.T + TB - 1) / TB;
    const long long nblk = (long long)n_tb * p.n_kv * p.n_seq;
    if (nblk > 0x7fffffff) return hipErrorNotSupported;
    ProfScope ps(kProfPrefill, st);
    if (p.ring_cap)
        hipLaunchKernelGGL((prefill_kernel<HD, RT, NW, true>), dim3((unsigned)nblk), dim3(64 * NW), 0, st, p, n_tb, TB);
    else
        hipLaunchKernelGGL((prefill_kernel<HD, RT, NW, false>), dim3((unsigned)nblk), dim3(64 * NW), 0, st, p, n_tb, TB);
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillParams& p, hipStream_t st) {
    if (p.hd == 64) return launch<64, 2, 4>(p, st);
    if (p.hd == 128) return launch<128, 1, 4>(p, st);
    return hipErrorNotSupported;
}

}  // namespace pelica
