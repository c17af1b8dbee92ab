// MLA (latent) attention for gfx950: one shared kv "head" whose keys and
// values are the same latent cache rows (512 f16 per position), f32
// absorbed queries [seq][token][head][512], f32 output — the mla kernel of
// src/gpu.rs:262-307 (called from src/forward.rs:936-960), as split-K
// flash-decode with an in-order combine.
//
// Work split.  A workgroup of 4 waves owns (sequence, row group of 16 query
// rows = (token, head) pairs, key split).  Latent blocks of 32 keys (32 KB)
// go from HBM straight into LDS (buffer_load ... lds, double buffered: ~74 KB
// of LDS, so two workgroups share a CU and one's loads and barriers hide
// behind the other's math); K = V, so each block is read from HBM once for
// both products (the row groups of a split read it through the same L2).
// Wave w owns dims [128 w, 128 w + 128): it computes the partial scores
// S_w^T = K[:, dims] Q[:, dims]^T on v_mfma_f32_16x16x32_f16 (Q split into
// f16 hi + lo parts, ~fp32 products), the four partials are summed through
// LDS, every wave runs the same online softmax (base 2), and wave w
// accumulates O^T[dims] += V^T[dims] P^T with V read by the transposing
// ds_read_b64_tr_b16 (P split into hi + lo as the B operand).  HBM-bound:
// per 32-key block 32 KB of latent against 128 MFMAs per wave.
#include <type_traits>

#include "attn_decode.hpp"
#include "attn_prof.hpp"

namespace pelica {

namespace {

constexpr int kBufFlags = 0x00020000;  // raw buffer, 32-bit format
constexpr int kMlaHd = 512;

// LDS byte offset of 16-byte piece p of key row k in a latent block: pieces
// XOR-swizzled by the key's low 4 bits so 16 consecutive keys read at one
// piece index hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ int mla_slot(int k, int p) { return k * (kMlaHd * 2) + ((p ^ (k & 15)) << 4); }

__device__ __forceinline__ const _Float16* mla_elem(const char* base, int k, int d) {
    return reinterpret_cast<const _Float16*>(base + mla_slot(k, d >> 3) + ((d & 7) << 1));
}

// s_waitcnt immediate: at most n vector-memory ops outstanding (gfx9
// encoding: vmcnt[3:0], expcnt[6:4] and lgkmcnt[11:8] left at max, vmcnt[5:4])
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

}  // namespace

// Build-time instrumentation (off by default; -DPELICA_MTRACE): lane 0 of
// wave 0 of each workgroup stores 100 MHz real-time stamps in
// g_mtrace[workgroup * 32 + k]: 0 entry; for block i < 7, 1 + 4 i at the
// loop top, 2 + 4 i once the block has landed (after the barrier), 3 + 4 i
// after the score exchange, 4 + 4 i after PV; 29 loop end, 30 stores done,
// 31 (XCC_ID << 32) | HW_ID (which CU ran it).  pelica_attn_debug_mtrace()
// copies them out.
#ifdef PELICA_MTRACE
__device__ unsigned long long g_mtrace[1 << 15];
#define MSTAMP(k)                                                                                          \
    do {                                                                                                   \
        if (tid == 0 && (k) < 32) g_mtrace[wg_lin * 32 + (k)] = __builtin_amdgcn_s_memrealtime();          \
    } while (0)
#else
#define MSTAMP(k) \
    do {          \
    } while (0)
#endif

template <int RT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void mla_kernel(DecodeParams p) {
    constexpr int HD = kMlaHd, NW = 4, KB = 32;  // dims, waves, keys per block
    constexpr int DS = HD / NW / 32;             // 32-dim k-steps per wave (4)
    constexpr int DT = HD / NW / 16;             // 16-dim output tiles per wave (8)
    constexpr int ROWS = 16 * RT, NP = 2;  // f16 parts of Q (hi + lo: ~fp32 scores)
    constexpr int NPP = 1;  // f16 parts of P (the PV weights: f16 alone is within tolerance)
    constexpr int BLK = KB * HD * 2;             // 32 KB
    constexpr int NBUF = 2;  // latent blocks in the LDS ring (two workgroups fit a CU's LDS)
    constexpr int LPB = KB / NW;                 // loads per block per thread
    constexpr int PS = KB + 4;  // partial-score row stride in floats: rows land on distinct banks
    __shared__ __attribute__((aligned(16))) char lds[NBUF * BLK + NW * ROWS * PS * 4];
    float* const part = reinterpret_cast<float*>(lds + NBUF * BLK);  // [NW][ROWS][PS] partial scores

    // (the wave index scalar: addresses built from it stay in SGPRs)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
              c16 = lane & 15;
    const int rg = blockIdx.y, s = blockIdx.z, slot = blockIdx.x;
#ifdef PELICA_MTRACE
    const int wg_lin = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    if (wg_lin >= 1024) return;
    if (tid == 0)
        g_mtrace[wg_lin * 32 + 31] = ((unsigned long long)__builtin_amdgcn_s_getreg(20 | (31 << 11)) << 32) |
                                     (unsigned)__builtin_amdgcn_s_getreg(4 | (31 << 11));
#endif
    MSTAMP(0);
    const int len = seq_keys(p.seq_len, s, p.kv_len);
    if (len < p.T || len <= 0) return;
    const int n_active = min(p.n_slot, (len - 1) / p.split_keys + 1);
    if (slot >= n_active) return;
    const int64_t row0 = p.seq_off ? p.seq_off[s] : (int64_t)s * p.kv_len;
    const int kbeg = slot * p.split_keys, kend = min(kbeg + p.split_keys, len);
    const int nblk = (kend - kbeg + KB - 1) / KB;
    const int rbase = rg * ROWS;

    const uint32_t stride_b = (uint32_t)p.row_stride * 2;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.k + row0 * p.row_stride), (short)0, (int)((uint32_t)len * stride_b), kBufFlags);
    // block i -> LDS buffer i % NBUF; wave instruction j of wave w fills key
    // row 4 j + w (64 slots of 16 bytes); the lane loads the piece its slot holds
    // (tracked: the prologue's loads, which the query loads are waited for
    // around; untracked: the loop's, see lds_dma16_untracked)
    auto load_block = [&](int i, bool tracked) {
        char* dst = lds + (i % NBUF) * BLK;
        const int kb = kbeg + KB * i;
#pragma unroll
        for (int j = 0; j < KB / NW; ++j) {
            const int key = NW * j + wave;
            const int piece = lane ^ (key & 15);
            const uint32_t off = (uint32_t)(kb + key) * stride_b + 16 * piece;
            if (tracked) lds_dma16(rs, off, dst + key * (HD * 2));
            else lds_dma16_untracked(rs, off, dst + key * (HD * 2));
        }
    };
    // queries of this lane's rows, this wave's dims (requested before the
    // first latent blocks, so waiting for them does not wait for the blocks)
    float4v qa[RT][DS], qb2[RT][DS];
    int posr[RT];
    bool qok[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = rbase + 16 * rt + c16;
        qok[rt] = r < p.R;
        const int rr = qok[rt] ? r : 0;
        const int t = rr / p.hpk, h = rr % p.hpk;
        const float* qp = p.q + (size_t)(s * p.T + t) * p.q_tok + h * HD + 128 * wave + 8 * g;
        posr[rt] = qok[rt] ? len - p.T + t : -1;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            qa[rt][ds] = *reinterpret_cast<const float4v*>(qp + 32 * ds);
            qb2[rt][ds] = *reinterpret_cast<const float4v*>(qp + 32 * ds + 4);
        }
    }
    if (nblk > 0) load_block(0, true);  // (a 2-block ring: the first fill is block 0)
    // f16 hi + lo parts, base 2
    half8 qf[NP][RT][DS];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = qok[rt] ? (j < 4 ? qa[rt][ds][j] : qb2[rt][ds][j - 4]) * p.qscale : 0.f;
                const _Float16 hi = (_Float16)x;
                qf[0][rt][ds][j] = hi;
                qf[1][rt][ds][j] = (_Float16)(x - (float)hi);
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

    // partial scores over this wave's dims: 2 key tiles x RT row tiles;
    // element e of (kt, rt) is key 16 kt + 4 g + e of row 16 rt + c16
    auto qk_part = [&](const char* blk, float4v (&pr)[2][RT]) {
        float4v acc[NP][2][RT];
#pragma unroll
        for (int pp = 0; pp < NP; ++pp)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) acc[pp][kt][rt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            half8 ka[2];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                ka[kt] = *reinterpret_cast<const half8*>(blk + mla_slot(16 * kt + c16, 16 * wave + 4 * ds + g));
#pragma unroll
            for (int pp = 0; pp < NP; ++pp)
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) acc[pp][kt][rt] = mfma16(ka[kt], qf[pp][rt][ds], acc[pp][kt][rt]);
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) pr[kt][rt] = acc[0][kt][rt] + acc[1][kt][rt];
    };
    auto write_part = [&](float* pb, const float4v (&pr)[2][RT]) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                *reinterpret_cast<float4v*>(pb + (wave * ROWS + 16 * rt + c16) * PS + 16 * kt + 4 * g) = pr[kt][rt];
    };
    auto read_sums = [&](const float* pb, float4v (&sc)[2][RT]) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                // (seeded with wave 0's partial: 0 + x is not x for x = -0)
                float4v t4 = *reinterpret_cast<const float4v*>(pb + (16 * rt + c16) * PS + 16 * kt + 4 * g);
#pragma unroll
                for (int w = 1; w < NW; ++w)
                    t4 += *reinterpret_cast<const float4v*>(pb + (w * ROWS + 16 * rt + c16) * PS + 16 * kt + 4 * g);
                sc[kt][rt] = t4;
            }
    };
    // causal mask (only the blocks that reach past a row's position or the
    // split) and online softmax, identical in every wave; the running max
    // moves (O and l rescaled) only when a row's block max exceeds it by
    // 2^8, so most blocks skip the rescale
    auto softmax = [&](int i, float4v (&sc)[2][RT], half8 (&pf)[NPP][RT]) {
        const int kb = kbeg + KB * i;
        if (kb + KB > kend || kb + KB - 1 > posr[0]) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int key = kb + 16 * kt + 4 * g + e;
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        if (key >= kend || key > posr[rt]) sc[kt][rt][e] = -INFINITY;
                }
        }
        float bm[RT];
        bool grow = false;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float x = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 4; ++e) x = fmaxf(x, sc[kt][rt][e]);
            bm[rt] = group4_max(x);
            grow |= bm[rt] > m[rt] + 8.f;
        }
        if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const float mn = fmaxf(m[rt], bm[rt]);
                if (mn > m[rt]) {
                    const float c = fast_exp2(m[rt] - mn);  // 0 when m was -inf
                    l[rt] *= c;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) o[dt][rt] *= c;
                    m[rt] = mn;
                }
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float ms = m[rt] == -INFINITY ? 0.f : m[rt];
            float ls = 0.f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float pe = fast_exp2(sc[kt][rt][e] - ms);
                    ls += pe;
                    const _Float16 hi = (_Float16)pe;
                    pf[0][rt][kt * 4 + e] = hi;
                    if (NPP > 1) pf[NPP - 1][rt][kt * 4 + e] = (_Float16)(pe - (float)hi);
                }
            l[rt] += ls;
        }
    };
    // O^T[this wave's dims] += V^T P^T (keys in the B operand's order)
    auto pv = [&](const char* blk, const half8 (&pf)[NPP][RT]) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int k0 = 4 * g + (c16 >> 2), d0 = 128 * wave + 16 * dt + 4 * (c16 & 3);
            const half8 va = cat8(lds_read_tr(mla_elem(blk, k0, d0)), lds_read_tr(mla_elem(blk, k0 + 16, d0)));
#pragma unroll
            for (int pp = 0; pp < NPP; ++pp)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) o[dt][rt] = mfma16(va, pf[pp][rt], o[dt][rt]);
        }
    };
    // s_waitcnt: block j is in LDS once at most the loads of the `later`
    // blocks issued after it are outstanding (loads complete in order)
    auto wait_later = [&](int later) {
        if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * LPB));
        else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPB));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    };

    // trip i on buffer PAR = i % 2, a compile-time constant (the loop is
    // unrolled by two): every LDS address is then a loop-invariant lane
    // offset plus an immediate
    auto trip = [&](auto par, int i) {
        constexpr int PAR = decltype(par)::value;
        const char* const blk = lds + PAR * BLK;
        if (i < 7) MSTAMP(1 + 4 * i);
        wait_later(min(nblk - 1 - i, NBUF - 2));
        lds_barrier();  // ... for every wave; block i-1's readers are done
        if (i < 7) MSTAMP(2 + 4 * i);
        if (i + 1 < nblk) load_block(i + 1, false);  // into block i-1's buffer
        float4v pr[2][RT];
        qk_part(blk, pr);
        write_part(part, pr);
        lds_barrier();
        float4v sc[2][RT];
        read_sums(part, sc);
        if (i < 7) MSTAMP(3 + 4 * i);
        half8 pf[NPP][RT];
        softmax(i, sc, pf);
        pv(blk, pf);
        if (i < 7) MSTAMP(4 + 4 * i);
    };
    for (int i = 0; i < nblk; i += 2) {
        trip(std::integral_constant<int, 0>{}, i);
        if (i + 1 < nblk) trip(std::integral_constant<int, 1>{}, i + 1);
    }
    MSTAMP(29);

    // this wave's dims of each row: the output, or the split's partial
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const float L = group4_sum(l[rt]);
        const int r = rbase + 16 * rt + c16;
        if (r >= p.R) continue;
        const int t = r / p.hpk, h = r % p.hpk;
        if (n_active == 1) {
            const float inv = 1.f / L;
            float* op = p.out + (size_t)(s * p.T + t) * p.o_tok + h * HD + 128 * wave + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<float4v*>(op + 16 * dt) = o[dt][rt] * inv;
        } else {
            const size_t idx = ((size_t)s * p.R + r) * p.n_slot + slot;
            if (wave == 0 && g == 0) *reinterpret_cast<float2*>(p.ws_ml + 2 * idx) = make_float2(m[rt], L);
            float* op = p.ws_o + idx * HD + 128 * wave + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<float4v*>(op + 16 * dt) = o[dt][rt];
        }
    }
#ifdef PELICA_MTRACE
    __builtin_amdgcn_s_waitcnt(0);
#endif
    MSTAMP(30);
}

#ifdef PELICA_MTRACE
extern "C" int pelica_attn_debug_mtrace(void* dst, size_t bytes) {
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_mtrace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

hipError_t launch_mla(const DecodeParams& p, hipStream_t st) {
    if (p.rg_rows != 16) return hipErrorInvalidValue;
    const dim3 grid(p.n_slot, p.n_rg, p.n_seq);
    {
        ProfScope ps(kProfDecodeSplit, st);
        hipLaunchKernelGGL(mla_kernel<1>, grid, dim3(256), 0, st, p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.n_slot == 1) return e;
    return launch_combine(p, st);
}

}  // namespace pelica
