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
#include <algorithm>
#include <type_traits>

#include "attn_prefill.hpp"
#include "attn_prof.hpp"

namespace pelica {

typedef float float16v __attribute__((ext_vector_type(16)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));

// word 3 of a gfx9 buffer resource: 32-bit data format, raw addressing
constexpr int kBufferFlags = 0x00020000;
// Cache policy of the query loads and output stores (each byte touched
// once).  Output stores go nt (streaming), so they do not displace the K/V
// the kv head's workgroups share in L2: the sliding-window kernel's
// window-128 prompt 26.5-26.6 -> 23.5-24.8 us (nt query loads as well:
// 26.9-28.1; nt query loads alone: 31.5-31.9), the full causal prompt
// 151.9-152.3 -> 150.8-151.4 us.
constexpr int kSlideLoadAux = 0, kSlideStoreAux = 2, kPreStoreAux = 2;

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

// waves per SIMD: 2 (64 query rows per wave at hd 64, 32 at hd 128), or 1
// with 128 rows per wave (the whole register file for one wave)
template <int HD, int RT>
constexpr int kPrefillOcc = HD * RT >= 256 ? 1 : 2;

// Build-time instrumentation (off by default; -DPELICA_PTRACE): per wave,
// shader-clock cycles spent in the tile loop, waiting for tile loads and at
// the per-chunk barrier, the number of exact-path chunks, and 100 MHz
// real-time stamps at entry, loop start, loop end and exit (their ratio to
// the cycle count gives the shader clock), and in the prologue after the
// query and tile loads are issued, after they landed and after the
// workgroup barrier, stored in g_ptrace[wave * 16 + k];
// pelica_attn_debug_ptrace() copies them out.
#ifdef PELICA_PTRACE
__device__ unsigned long long g_ptrace[1 << 18];
__device__ __forceinline__ unsigned cyc() { return (unsigned)__builtin_amdgcn_s_memtime(); }
__device__ __forceinline__ unsigned long long rtime() { return __builtin_amdgcn_s_memrealtime(); }
#endif

// Short key ranges (sliding windows): with NRES > 0 every K and V tile of
// the workgroup's range (at most NRES of each) is requested at the start and
// stays resident in LDS, so the chunk loop has no tile waits and no
// barriers; otherwise tiles stream through two K and two V buffers.
// F32: f32 queries (rounded to f16 as they are loaded) and f32 output.
template <int HD, int RT, bool RING, bool ROUND, int NW, int NRES = 0, bool F32 = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(kPrefillOcc<HD, RT>, kPrefillOcc<HD, RT>))) void prefill_kernel(
    PrefillParams p, int n_tb, int TB) {
    constexpr int KS = HD / 16;                 // 16-dim k-steps of QK^T
    constexpr int DT = HD / 32;                 // 32-dim output tiles
    constexpr int TILE = 64 * HD * 2;           // bytes of a 64-key K (or V) tile
    constexpr int PPR = HD / 8;                 // 16-byte pieces per key row
    // streaming: K0 K1 V0 V1; resident: K[NRES] V[NRES] and a zero tile
    constexpr int NBUF = NRES ? 2 * NRES + 1 : 4;
    static_assert(!NRES || !ROUND, "resident tiles: whole-cache launches only");
    // after the tile loop the f16 output of each wave is staged here
    constexpr int OUT_WAVE = RT * 32 * HD * 2;  // bytes of one wave's output rows
    constexpr int LDS_BYTES = (ROUND || NBUF * TILE >= NW * OUT_WAVE) ? NBUF * TILE : NW * OUT_WAVE;
    __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];

    // XCD-aware block order: dispatch goes round-robin over the 8 XCDs, so
    // give each XCD a contiguous range of logical blocks (same kv head)
    const int nblk = gridDim.x;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int tb = n_tb - 1 - bid % n_tb;  // longest key ranges first
    const int rest = bid / n_tb;
    const int kvh = rest % p.n_kv, s = rest / p.n_kv;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h2 = lane >> 5, c32 = lane & 31;
#ifdef PELICA_PTRACE
    const unsigned long long rt_entry = rtime();
    unsigned long long rt_loop0 = 0, rt_loop1 = 0, rt_issued = 0, rt_landed = 0, rt_bar = 0;
#endif
    const int len = seq_keys(p.seq_len, s, p.kv_len);
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
    // keys this launch covers: the whole cache, or one round's rows
    const int kbeg = ROUND ? p.key_begin : 0, kend = ROUND ? min(p.key_end, len) : len;
    const uint32_t stride_b = (uint32_t)p.row_stride * 2;
    const uint32_t nrec = (RING ? (uint32_t)p.ring_cap : (uint32_t)(kend - kbeg)) * stride_b;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.k + row0 * p.row_stride + (size_t)kvh * HD), (short)0, (int)nrec, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.v + row0 * p.row_stride + (size_t)kvh * HD), (short)0, (int)nrec, kBufferFlags);
    // 32-key chunks from the first chunk any row sees to the last: tiles of
    // 64 keys start at kb0 (32-aligned), and the last tile may hold only one
    // needed chunk (a 32-token block of a window-128 layer takes 5 chunks, not
    // the 6 of 64-aligned whole tiles)
    const int kb0 = max(lo_first, kbeg) & ~31;
    const int klast = min(pos_last, kend - 1);
    const int n_chunks = klast >= kb0 ? (klast - kb0) / 32 + 1 : 0;  // 0: a round past these tokens
    const int n_tiles = (n_chunks + 1) / 2;
    // Tiles go from HBM straight into LDS (buffer_load ... lds): wave
    // instruction i of wave w fills LDS slots 64 (NW i + w) + lane (16 bytes
    // each) of a tile; the lane loads the logical piece that the swizzled
    // layout puts in its slot.
    constexpr int WI = PPR / NW;  // wave instructions per tile and wave
    static_assert(PPR % NW == 0, "tile pieces must split evenly over the waves");
    char* const kbuf = lds;                            // K tiles
    char* const vbuf = lds + (NRES ? NRES : 2) * TILE;  // V tiles
    // buffer of tile t: its own (resident) or t & 1 (streaming)
    auto tbuf = [](int t) { return NRES ? t : (t & 1); };
    // tracked: the prologue's loads; the chunk loop's are untracked (the
    // compiler would wait for them before the PV's transposing V reads of
    // the same chunk; the loop waits for them itself, at the next barrier)
    auto load_tile = [&](const __amdgpu_buffer_rsrc_t& rs, char* dst, int tile, bool is_v, bool tracked) {
        const int kb = kb0 + 64 * tile;
#pragma unroll
        for (int i = 0; i < WI; ++i) {
            const int slot = 64 * (NW * i + wave) + lane;
            const int key = slot / PPR, phys = slot % PPR;
            const int piece = is_v ? phys ^ ((key & 3) << 1) : phys ^ (key & 7);
            // (round rows before key_begin wrap to offsets past nrec: zeros)
            const uint32_t off = RING ? ((kb + key) % p.ring_cap) * stride_b + 16 * piece
                                      : (uint32_t)(kb + key - kbeg) * stride_b + 16 * piece;
            if (tracked) lds_dma16(rs, off, dst + 1024 * (NW * i + wave));
            else lds_dma16_untracked(rs, off, dst + 1024 * (NW * i + wave));
        }
    };
    // s_waitcnt vmcnt(0): the tile loads above have landed in LDS
    auto wait_tiles = [] { __builtin_amdgcn_s_waitcnt(0x0F70); };

    // The first tiles are requested before anything else, and nothing in
    // the prologue after them waits for a load: the queries come through a
    // buffer resource whose out-of-range offsets read as zeros (rows past
    // the block need no select on loaded data) and the sink logits are
    // loaded for every row.  (A select or a conditional load there makes
    // the compiler wait for every load issued before it — with the tile
    // requests behind it, a whole HBM round trip.)
    // the (empty) PV of chunk -1 reads this zeroed tile: V tile 1's
    // buffer (streaming) or the tile after the resident ones
    char* const vzero = NRES ? lds + 2 * NRES * TILE : vbuf + TILE;
    if (n_tiles > 0) {  // (uniform over the workgroup)
#pragma unroll
        for (int i = 0; i < TILE / (16 * 64 * NW); ++i)
            *reinterpret_cast<u32x4*>(vzero + 16 * (tid + 64 * NW * i)) = u32x4{0, 0, 0, 0};
        if (NRES) {
            // (the launch guarantees n_tiles <= NRES)
            for (int t = 0; t < n_tiles; ++t) load_tile(rk, kbuf + t * TILE, t, false, true);
            for (int t = 0; t < n_tiles; ++t) load_tile(rv, vbuf + t * TILE, t, true, true);
        } else {
            load_tile(rk, kbuf, 0, false, true);
            if (n_tiles > 1) load_tile(rk, kbuf + TILE, 1, false, true);
            load_tile(rv, vbuf, 0, true, true);
        }
    }

    // this lane's query rows (column c32 of each 32-row tile): Q as the B
    // operand, position and window start
    half8 qb[RT][KS];
    int posr[RT], lor[RT];
    bool valid[RT];
    constexpr int QES = F32 ? 4 : 2;                      // bytes per query / output value
    const uint32_t qtok_b = (uint32_t)p.q_tok * QES;      // bytes between consecutive tokens' queries
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const char*>(p.q) + ((size_t)s * p.T + t0) * p.q_tok * QES), (short)0,
        (int)((uint32_t)(t1 - t0) * qtok_b), kBufferFlags);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = (wave * RT + rt) * 32 + c32;
        const int t = t0 + r / p.hpk;
        valid[rt] = r < TB * p.hpk && t < t1;
        const int h = kvh * p.hpk + r % p.hpk;
        const uint32_t qoff = valid[rt] ? (uint32_t)(t - t0) * qtok_b + (uint32_t)(h * HD + 8 * h2) * QES : 0xFFFFFF00u;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if constexpr (F32) {
                const float4v a = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + 64 * ks, 0, 0));
                const float4v b = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + 64 * ks + 16, 0, 0));
                qb[rt][ks] = half8{(_Float16)a[0], (_Float16)a[1], (_Float16)a[2], (_Float16)a[3],
                                   (_Float16)b[0], (_Float16)b[1], (_Float16)b[2], (_Float16)b[3]};
            } else {
                qb[rt][ks] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + 32 * ks, 0, 0));
            }
        }
        posr[rt] = valid[rt] ? len - p.T + t : -1;
        lor[rt] = (p.window > 0 && posr[rt] + 1 > p.window) ? posr[rt] + 1 - p.window : 0;
    }

    // running state; a sink starts it at (max = sink, sum = 1)
    float m[RT], l[RT];
    float16v o[DT][RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m[rt] = valid[rt] ? -INFINITY : 0.f;  // rows past the block: all masked, fast path
        l[rt] = 0.f;
        if (!ROUND && p.sinks) {  // (every row's index is a head of this kv head)
            const int r = (wave * RT + rt) * 32 + c32;
            const float sk = p.sinks[kvh * p.hpk + r % p.hpk] * kLog2e;
            m[rt] = valid[rt] ? sk : m[rt];
            l[rt] = valid[rt] && h2 == 0 ? 1.f : 0.f;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt][rt] = float16v{};
        if (ROUND && !p.first && valid[rt]) {
            // the running state of the rounds before (sum split over h2 lanes)
            const int r = (wave * RT + rt) * 32 + c32;
            const int t = t0 + r / p.hpk, h = kvh * p.hpk + r % p.hpk;
            const float* st = p.state + ((size_t)(s * p.T + t) * p.n_head + h) * (HD + 2);
            m[rt] = st[0] <= -1.0e38f ? -INFINITY : st[0] * kLog2e;
            l[rt] = h2 == 0 ? st[1] : 0.f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][rt][i] = st[2 + 32 * dt + 8 * (i / 4) + 4 * h2 + i % 4];
        }
    }

    // S^T of chunk c (32 keys x RT row tiles): element i of a lane is key
    // 32 c + 8 (i / 4) + 4 h2 + i % 4 of row c32
    auto qk = [&](int c, float16v (&sc)[RT]) {
        const char* kt = kbuf + tbuf(c >> 1) * TILE;
        const int krow = 32 * (c & 1) + c32;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sc[rt] = float16v{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const half8 ka = *reinterpret_cast<const half8*>(kt + k_slot<HD>(krow, 2 * ks + h2));
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) sc[rt] = mfma32(ka, qb[rt][ks], sc[rt]);
        }
    };
    // O^T += V^T P^T over chunk c; pb[w] holds keys 16 w .. 16 w + 15 of it
    auto pv = [&](int c, const half8 (&pb)[2][RT]) {
        const char* vt = vbuf + tbuf(c >> 1) * TILE;
        const int G = lane >> 4, r4 = (lane & 15) >> 2, q4 = lane & 3;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            half8 va[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                // lanes of 16-lane group G read keys 16w + 4 h2 + r (+8) at
                // dims 32 dt + 16 (G & 1) + 4 q; lane 4r + q of the group
                const int key = 32 * (c & 1) + 16 * w + 4 * h2 + r4, dim = 32 * dt + 16 * (G & 1) + 4 * q4;
                const _Float16* a0 = reinterpret_cast<const _Float16*>(vt + v_slot<HD>(key, dim >> 3) + ((dim & 7) << 1));
                const _Float16* a1 = reinterpret_cast<const _Float16*>(vt + v_slot<HD>(key + 8, dim >> 3) + ((dim & 7) << 1));
                va[dt] = cat8(lds_read_tr(a0), lds_read_tr(a1));
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) o[dt][rt] = mfma32(va[dt], pb[w][rt], o[dt][rt]);
        }
    };

    // Software pipeline over 32-key chunks: while the softmax of chunk c
    // runs on the vector ALUs, the matrix cores take QK^T of chunk c+1 and
    // PV of chunk c-1.  K tiles and V tiles are double-buffered separately;
    // one barrier per 64-key tile orders the tile loads against their
    // readers.
    //
    // Softmax without a per-chunk max: P = 2^(s*scale - m) with the running
    // m; a lane whose chunk sum stays <= 2^14 had no overflow or loss (every
    // P is <= its sum, f16 keeps 11 bits at any magnitude), and once m is
    // some key's score (or the sink) that key's own term keeps l >= 1, so
    // terms flushed to 0 are negligible.  Otherwise (no max yet, a new
    // maximum far above m) the wave takes the exact path: chunk max, rescale
    // O and l, recompute P.
    constexpr float kSumLimit = 16384.f;
    if (n_tiles > 0) {  // (uniform over the workgroup)
    {
#ifdef PELICA_PTRACE
        rt_issued = rtime();
#endif
        wait_tiles();
#ifdef PELICA_PTRACE
        rt_landed = rtime();
#endif
    }
    __syncthreads();
#ifdef PELICA_PTRACE
    rt_bar = rtime();
#endif

#ifdef PELICA_PTRACE
    unsigned t_wait = 0, t_bar = 0, n_exact = 0;
#endif
    float16v s_a[RT], s_b[RT];
    half8 p_a[2][RT], p_b[2][RT];
#pragma unroll
    for (int w = 0; w < 2; ++w)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) p_b[w][rt] = half8{0, 0, 0, 0, 0, 0, 0, 0};
    qk(0, s_a);
    const half2 one2 = {(_Float16)1.f, (_Float16)1.f};

    // one chunk: scores of c in s_cur, of c+1 into s_nxt; P of c-1 in
    // p_prv, of c into p_cur
    // PAR = c mod 4 as a compile-time constant: it picks the K/V tile
    // buffers, so every LDS operand address is a loop-invariant lane offset
    // plus an immediate.
    auto step = [&](auto par, int c, float16v (&s_cur)[RT], float16v (&s_nxt)[RT], const half8 (&p_prv)[2][RT],
                    half8 (&p_cur)[2][RT]) {
        constexpr int PAR = decltype(par)::value;
        // K of tile t+2 and V of tile t+1 at odd chunks c = 2t+1: their
        // buffers' last readers finished at chunk 2t; first readers at 2t+3
        const int t = c >> 1;
        if (!NRES && (PAR & 1)) {
            if (t + 2 < n_tiles) load_tile(rk, kbuf + (t & 1) * TILE, t + 2, false, false);
            if (t + 1 < n_tiles) load_tile(rv, vbuf + ((t + 1) & 1) * TILE, t + 1, true, false);
        }

        const int kb = kb0 + 32 * c;
        if (kb + 31 > pos_first || kb < lo_last || (ROUND && (kb < kbeg || kb + 31 >= kend))) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kb + 8 * (i / 4) + 4 * h2 + (i % 4);
                const bool out_of_round = ROUND && (key < kbeg || key >= kend);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    if (key < lor[rt] || key > posr[rt] || out_of_round) s_cur[rt][i] = -INFINITY;
            }
        }

        // operands: KS K pieces of QK^T (chunk c+1, past the last chunk:
        // discarded), then 2 DT V pieces of PV (chunk c-1); each read two
        // operands ahead of its first MFMA
        constexpr int NOPD = KS + 2 * DT;
        half8 opd[NOPD];
        // (resident tiles: PAR = c itself)
        const char* const kt_c = kbuf + (NRES ? ((PAR + 1) >> 1) : (((PAR + 1) >> 1) & 1)) * TILE;
        const int krow = 32 * ((PAR + 1) & 1) + c32;
        // chunk c-1 (c = 0: the zeroed tile)
        const char* const vt_c = NRES ? (PAR == 0 ? vzero : vbuf + ((PAR - 1) >> 1) * TILE)
                                      : vbuf + (((PAR + 3) >> 1) & 1) * TILE;
        auto read_opd = [&](int r) {
            if (r < KS) {
                opd[r] = *reinterpret_cast<const half8*>(kt_c + k_slot<HD>(krow, 2 * r + h2));
            } else {
                // lanes of 16-lane group G read keys 16w + 4 h2 + r4 (+8) at
                // dims 32 dt + 16 (G & 1) + 4 q4; lane 4 r4 + q4 of the group
                const int w = (r - KS) / DT, dt = (r - KS) % DT;
                const int G = lane >> 4, r4 = (lane & 15) >> 2, q4 = lane & 3;
                const int key = 32 * ((PAR + 3) & 1) + 16 * w + 4 * h2 + r4, dim = 32 * dt + 16 * (G & 1) + 4 * q4;
                const _Float16* a0 = reinterpret_cast<const _Float16*>(vt_c + v_slot<HD>(key, dim >> 3) + ((dim & 7) << 1));
                const _Float16* a1 = reinterpret_cast<const _Float16*>(vt_c + v_slot<HD>(key + 8, dim >> 3) + ((dim & 7) << 1));
                opd[r] = cat8(lds_read_tr(a0), lds_read_tr(a1));
            }
        };
        read_opd(0);
        read_opd(1);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) s_nxt[rt] = float16v{};

        // The wave's MFMAs (QK^T of c+1, then PV of c-1) interleaved in
        // program order with the softmax of chunk c, so the matrix cores and
        // the vector ALUs work side by side.  The softmax runs as four
        // stages (fma, exp2, f16 pack, row-sum dot) skewed by one MFMA slot
        // each: slot t takes the fmas of scores S(t+1).., the exp2s of
        // scores S t.., the packs of the pairs exp'd in slot t-1 and the
        // dots of the pairs packed in slot t-1, so every 32-cycle MFMA has
        // the same small mix of vector work beside it (S scores per slot).
        constexpr int NM = KS * RT + 2 * DT * RT;  // MFMAs
        constexpr int NS = 16 * RT;                // scores per lane
        constexpr int NP = NS / 2;                 // score pairs
        static_assert(NS % NM == 0, "whole scores per MFMA slot");
        constexpr int S = NS / NM;
        // y = s*scale - ms in place (ms: the running max, 0 while it is -inf,
        // so the exact path below can recover s*scale = y + ms)
        float ms[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) ms[rt] = m[rt] == -INFINITY ? 0.f : m[rt];
        float acc[RT][2];
        float e[NS];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt][0] = acc[rt][1] = 0.f;
        auto op_fma = [&](int i) {
            if (i < NS) s_cur[i / 16][i % 16] = __builtin_fmaf(s_cur[i / 16][i % 16], p.qscale, -ms[i / 16]);
        };
        auto op_exp = [&](int i) {
            if (i < NS) e[i] = fast_exp2(s_cur[i / 16][i % 16]);
        };
        auto op_pack = [&](int k) {
            const int rt = k / 8, i = 2 * (k % 8);
            p_cur[i / 8][rt][i % 8] = (_Float16)e[2 * k];
            p_cur[i / 8][rt][i % 8 + 1] = (_Float16)e[2 * k + 1];
        };
        auto op_dot = [&](int k) {
            const int rt = k / 8, i = 2 * (k % 8);
            acc[rt][k & 1] = __builtin_amdgcn_fdot2(half2{p_cur[i / 8][rt][i % 8], p_cur[i / 8][rt][i % 8 + 1]}, one2,
                                                    acc[rt][k & 1], false);
        };
        // pairs whose both exp2s are done after slot u: (S (u + 1)) / 2
        auto packable = [](int u) { return u < 0 ? 0 : (S * (u + 1)) / 2; };
#pragma unroll
        for (int j = 0; j < S; ++j) op_fma(j);
#pragma unroll
        for (int t = 0; t < NM; ++t) {
            const int r = t / RT;  // operand of MFMA t
            if (t % RT == 0 && r + 2 < NOPD) read_opd(r + 2);
            // 8-wave workgroups: the wave about to issue its MFMA takes
            // issue priority over its SIMD partner's vector work (the
            // 4096-token gpt-oss causal prefill ~1.7 % faster; 4-wave
            // window launches ~3 % slower with it)
            if (NW == 8) __builtin_amdgcn_s_setprio(3);
            if (t < KS * RT) {
                const int rt = t % RT;
                s_nxt[rt] = mfma32(opd[r], qb[rt][r], s_nxt[rt]);
            } else {
                const int j = t - KS * RT, w = j / (DT * RT), dt = (j / RT) % DT, rt = j % RT;
                o[dt][rt] = mfma32(opd[r], p_prv[w][rt], o[dt][rt]);
            }
            if (NW == 8) __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int k = packable(t - 3); k < packable(t - 2); ++k) op_dot(k);
#pragma unroll
            for (int k = packable(t - 2); k < packable(t - 1); ++k) op_pack(k);
#pragma unroll
            for (int j = 0; j < S; ++j) op_exp(S * t + j);
#pragma unroll
            for (int j = 0; j < S; ++j) op_fma(S * (t + 1) + j);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int k = packable(NM - 2); k < NP; ++k) op_pack(k);
#pragma unroll
        for (int k = packable(NM - 3); k < NP; ++k) op_dot(k);
        float ls[RT];
        bool bad = false;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            ls[rt] = acc[rt][0] + acc[rt][1];
            bad |= !(ls[rt] <= kSumLimit) || m[rt] == -INFINITY;  // no max yet: the exact path sets it
        }
        if (__builtin_amdgcn_ballot_w64(bad)) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                // s*scale = y + ms
                float x = -INFINITY;
#pragma unroll
                for (int i = 0; i < 16; ++i) x = fmaxf(x, s_cur[rt][i]);
                const float mn = fmaxf(m[rt], half_max(x) + ms[rt]);
                if (mn > m[rt]) {
                    const float cf = fast_exp2(m[rt] - mn);  // 0 when m was -inf
                    l[rt] *= cf;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) o[dt][rt] *= cf;
                    m[rt] = mn;
                }
                const float shift = ms[rt] - (m[rt] == -INFINITY ? 0.f : m[rt]);
                float a = 0.f;
#pragma unroll
                for (int w = 0; w < 2; ++w)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        p_cur[w][rt][j] = (_Float16)fast_exp2(s_cur[rt][8 * w + j] + shift);
                        a += (float)p_cur[w][rt][j];
                    }
                ls[rt] = a;
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) l[rt] += ls[rt];
        // One barrier per tile, after its even chunk c = 2t: (a) the loads
        // issued at chunk 2t+1 overwrite buffers whose last readers ran at
        // chunk 2t, and (b) the loads of chunk 2t-1 are first read at chunk
        // 2t+1, so they must have landed (vmcnt(0)) before it.  Chunk 2t+1
        // reads only tiles published by this barrier or earlier ones.
        if (!NRES && (PAR & 1) == 0) {
#ifdef PELICA_PTRACE
            const unsigned ta = cyc();
            wait_tiles();
            const unsigned tb2 = cyc();
            __syncthreads();
            t_wait += tb2 - ta;
            t_bar += cyc() - tb2;
#else
            wait_tiles();
            __syncthreads();
#endif
        }
#ifdef PELICA_PTRACE
        n_exact += __builtin_amdgcn_ballot_w64(bad) != 0;
#endif
    };
#ifdef PELICA_PTRACE
    const unsigned t_start = cyc();
    rt_loop0 = rtime();
#endif
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P3 = std::integral_constant<int, 3>;
    if constexpr (NRES > 0) {
        // every chunk unrolled (n_chunks <= 2 NRES); PAR = c
        static_assert(NRES <= 4, "unrolled chunk steps");
        using P4 = std::integral_constant<int, 4>;
        using P5 = std::integral_constant<int, 5>;
        using P6 = std::integral_constant<int, 6>;
        using P7 = std::integral_constant<int, 7>;
        step(P0{}, 0, s_a, s_b, p_b, p_a);
        if (n_chunks > 1) step(P1{}, 1, s_b, s_a, p_a, p_b);
        if (n_chunks > 2) step(P2{}, 2, s_a, s_b, p_b, p_a);
        if (n_chunks > 3) step(P3{}, 3, s_b, s_a, p_a, p_b);
        if (NRES > 2 && n_chunks > 4) step(P4{}, 4, s_a, s_b, p_b, p_a);
        if (NRES > 2 && n_chunks > 5) step(P5{}, 5, s_b, s_a, p_a, p_b);
        if (NRES > 3 && n_chunks > 6) step(P6{}, 6, s_a, s_b, p_b, p_a);
        if (NRES > 3 && n_chunks > 7) step(P7{}, 7, s_b, s_a, p_a, p_b);
        // P of the last chunk: p_a after an even chunk, p_b after an odd one
        if (n_chunks & 1) pv(n_chunks - 1, p_a);
        else pv(n_chunks - 1, p_b);
    } else {
    int c = 0;
    for (; c + 4 <= n_chunks; c += 4) {
        step(P0{}, c, s_a, s_b, p_b, p_a);
        step(P1{}, c + 1, s_b, s_a, p_a, p_b);
        step(P2{}, c + 2, s_a, s_b, p_b, p_a);
        step(P3{}, c + 3, s_b, s_a, p_a, p_b);
    }
    // the last 1-3 chunks; P of the last chunk ends in p_a after an even
    // chunk count's odd step and in p_b after an even step
    const int rem = n_chunks - c;
    if (rem >= 1) step(P0{}, c, s_a, s_b, p_b, p_a);
    if (rem >= 2) step(P1{}, c + 1, s_b, s_a, p_a, p_b);
    if (rem >= 3) step(P2{}, c + 2, s_a, s_b, p_b, p_a);
    if (rem & 1) pv(n_chunks - 1, p_a);
    else pv(n_chunks - 1, p_b);
    }
#ifdef PELICA_PTRACE
    rt_loop1 = rtime();
    if (lane == 0) {
        const int wid = blockIdx.x * NW + wave;
        g_ptrace[wid * 16 + 0] = cyc() - t_start;
        g_ptrace[wid * 16 + 1] = t_wait;
        g_ptrace[wid * 16 + 2] = t_bar;
        g_ptrace[wid * 16 + 3] = (unsigned long long)n_exact << 32 | (unsigned)n_chunks;
    }
#endif
    }

    if constexpr (!ROUND && F32) {
        // f32 output: each lane stores its rows' 16-byte pieces
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float inv = 1.f / half_sum(l[rt]);
            if (!valid[rt]) continue;
            const int r = (wave * RT + rt) * 32 + c32;
            const int t = t0 + r / p.hpk, h = kvh * p.hpk + r % p.hpk;
            float* op = static_cast<float*>(p.out) + (size_t)(s * p.T + t) * p.o_tok + h * HD + 4 * h2;
            // O^T lane layout: dim 32 dt + 8 (i / 4) + 4 h2 + i % 4 of row c32
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4)
                    *reinterpret_cast<float4v*>(op + 32 * dt + 8 * i4) =
                        float4v{o[dt][rt][4 * i4], o[dt][rt][4 * i4 + 1], o[dt][rt][4 * i4 + 2], o[dt][rt][4 * i4 + 3]} * inv;
        }
    } else if constexpr (!ROUND) {
        // Output through LDS: each wave writes its rows (normalised, f16)
        // into its own area, then stores whole rows — consecutive rows are
        // consecutive heads of a token, so one store instruction writes
        // 512 B (hd 64) of contiguous output instead of 16-byte pieces of
        // 32 rows.  Rows of 16-byte pieces, piece p of local row r at slot
        // p ^ (r % PPR).
        __syncthreads();  // every wave is done with the K/V tiles
        char* const ow = lds + wave * OUT_WAVE;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float inv = 1.f / half_sum(l[rt]);
            const int rl = rt * 32 + c32;
            // O^T lane layout: dim 32 dt + 8 (i / 4) + 4 h2 + i % 4 of row c32
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const half4 hv = {(_Float16)(o[dt][rt][4 * i4] * inv), (_Float16)(o[dt][rt][4 * i4 + 1] * inv),
                                      (_Float16)(o[dt][rt][4 * i4 + 2] * inv), (_Float16)(o[dt][rt][4 * i4 + 3] * inv)};
                    const int pc = 4 * dt + i4;
                    *reinterpret_cast<half4*>(ow + rl * (HD * 2) + ((pc ^ (rl % PPR)) << 4) + 8 * h2) = hv;
                }
        }
        // (a wave's LDS accesses complete in order: it reads its own rows)
        // Every row is read back first, then stored through a buffer
        // resource over the block's output tokens: rows past the block fall
        // outside it (offset past num_records) and are dropped, no branch
        // per store.
        constexpr int RPI = 64 / PPR;  // rows per store instruction
        constexpr int NST = RT * 32 / RPI;
        const int pc = lane % PPR;
        u32x4 val[NST];
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            const int rl = k * RPI + lane / PPR;
            val[k] = *reinterpret_cast<const u32x4*>(ow + rl * (HD * 2) + ((pc ^ (rl % PPR)) << 4));
        }
        const uint32_t otok_b = (uint32_t)p.o_tok * 2;
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(static_cast<uint16_t*>(p.out) + ((size_t)s * p.T + t0) * p.o_tok), (short)0,
            (int)((uint32_t)(t1 - t0) * otok_b), kBufferFlags);
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            const int r = wave * RT * 32 + k * RPI + lane / PPR;
            const uint32_t off = r < TB * p.hpk ? (uint32_t)(r / p.hpk) * otok_b +
                                                      (uint32_t)((kvh * p.hpk + r % p.hpk) * HD + 8 * pc) * 2
                                                : 0xFFFFFF00u;  // (rows past the block's token count)
            __builtin_amdgcn_raw_buffer_store_b128(val[k], ro, off, 0, kPreStoreAux);
        }
    } else {
    // O^T lane layout: dim 32 dt + 8 (i / 4) + 4 h2 + i % 4 of row c32
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const float lt = half_sum(l[rt]);
        if (!valid[rt]) continue;
        const int r = (wave * RT + rt) * 32 + c32;
        const int t = t0 + r / p.hpk, h = kvh * p.hpk + r % p.hpk;
        float inv = 1.f / lt;
        if (ROUND) {
            float* st = p.state + ((size_t)(s * p.T + t) * p.n_head + h) * (HD + 2);
            if (h2 == 0) {
                st[0] = m[rt] == -INFINITY ? -3.0e38f : m[rt] * kLn2;
                st[1] = lt;
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) st[2 + 32 * dt + 8 * (i / 4) + 4 * h2 + i % 4] = o[dt][rt][i];
            if (!p.out) continue;
            // the output so far: sink in max and denominator; 0 before any key
            if (p.sinks) {
                const float sk = p.sinks[h] * kLog2e;
                const float M2 = fmaxf(m[rt], sk);
                const float w = m[rt] == -INFINITY ? 0.f : fast_exp2(m[rt] - M2);
                inv = w / (lt * w + fast_exp2(sk - M2));
            } else {
                inv = lt > 0.f ? inv : 0.f;
            }
        }
        const size_t obase = (size_t)(s * p.T + t) * p.o_tok + h * HD + 4 * h2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const float4v ov = float4v{o[dt][rt][4 * i4], o[dt][rt][4 * i4 + 1], o[dt][rt][4 * i4 + 2],
                                           o[dt][rt][4 * i4 + 3]} * inv;
                if constexpr (F32) {
                    *reinterpret_cast<float4v*>(static_cast<float*>(p.out) + obase + 32 * dt + 8 * i4) = ov;
                } else {
                    const half4 hv = {(_Float16)ov[0], (_Float16)ov[1], (_Float16)ov[2], (_Float16)ov[3]};
                    *reinterpret_cast<half4*>(static_cast<uint16_t*>(p.out) + obase + 32 * dt + 8 * i4) = hv;
                }
            }
    }
    }
#ifdef PELICA_PTRACE
    // (stores issued; the wave ends when they are done)
    if (lane == 0) {
        const int wid = blockIdx.x * NW + wave;
        g_ptrace[wid * 16 + 4] = rt_entry;
        g_ptrace[wid * 16 + 5] = rt_loop0;
        g_ptrace[wid * 16 + 6] = rt_loop1;
        g_ptrace[wid * 16 + 7] = rtime();
        g_ptrace[wid * 16 + 8] = rt_issued;
        g_ptrace[wid * 16 + 9] = rt_landed;
        g_ptrace[wid * 16 + 10] = rt_bar;
        g_ptrace[wid * 16 + 15] = 0;  // (this kernel's layout)
    }
#endif
}

// Sliding-window prefill over consecutive token blocks (head dim 64, 8
// heads per kv head, windows up to 130 keys, linear or ring caches).  One
// 8-wave workgroup per CU
// takes `spw` consecutive 64-token blocks of one kv head.  Keys sit in LDS
// as a ring of 32-key chunks (slot = chunk mod NCH): consecutive blocks
// share all but their last two chunks, so a block brings in two new chunks
// (8 KB of K and V) and its queries, both requested while the block before
// it is computed — its queries through the wave's own 8 KB staging area,
// which also stages that wave's output rows.  Each wave walks only the
// chunks its 8 tokens see (5 or 6); chunks are resident, so the chunk loop
// has no waits or barriers; one barrier per block hands the ring over.
// The chunk step is the one of prefill_kernel (same pipeline, same lazy
// softmax), with ring addresses in place of tile buffers.
template <int NCH, bool RING>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_slide_kernel(
    PrefillParams p, int n_parts, int spw) {
    constexpr int HD = 64, RT = 2, NW = 8, KS = HD / 16, DT = HD / 32, PPR = HD / 8, HPK = 8;
    constexpr int CHB = 32 * HD * 2;            // bytes of a 32-key chunk of K (or V)
    constexpr int OUT_WAVE = RT * 32 * HD * 2;  // bytes of one wave's rows (queries in, output out)
    constexpr int TBK = NW * RT * 32 / HPK;     // tokens per block (64)
    __shared__ __attribute__((aligned(16))) char lds[2 * NCH * CHB + CHB + NW * OUT_WAVE];
    char* const kring = lds;
    char* const vring = lds + NCH * CHB;
    char* const vzero = lds + 2 * NCH * CHB;  // the (empty) PV of chunk -1 reads zeros

    const int nblk = gridDim.x;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);  // one kv head per XCD
    const int part = bid % n_parts, rest = bid / n_parts;
    const int kvh = rest % p.n_kv, s = rest / p.n_kv;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, h2 = lane >> 5,
              c32 = lane & 31;
    char* const stage = vzero + CHB + wave * OUT_WAVE;
#ifdef PELICA_PTRACE
    // stamps (prefill_kernel's layout where they mean the same): [0]
    // compute cycles, [1] block-top wait cycles, [2] barrier cycles, [3]
    // exact-path chunks << 32 | chunks, [4] entry, [5] first compute start,
    // [6] last compute end, [7] exit, [8] + 2 k / [9] + 2 k: compute start /
    // end of the workgroup's block k (k < 3), for block 1: [12] barrier
    // passed, [13] queries read, [14] previous output stored; [15] = 1
    // (this kernel's layout)
    const unsigned long long rt_entry = rtime();
    unsigned t_comp = 0, t_wait = 0, t_bar = 0, n_ch_all = 0, n_exact = 0;
    unsigned long long rt_first = 0, rt_last = 0;
    const int wid = blockIdx.x * 8 + (threadIdx.x >> 6);
#endif
    // the lane index through an empty asm: per-block address arithmetic
    // derived from it is recomputed where it is used instead of being
    // hoisted out of the block loop (where it would hold ~40 VGPRs)
    auto fresh_lane = [&] {
        int ln = lane;
        __asm__ volatile("" : "+v"(ln));
        return ln;
    };

    const int len = seq_keys(p.seq_len, s, p.kv_len);
    if (len < p.T || len <= 0) return;
    const int n_steps = (p.T + TBK - 1) / TBK;
    const int j0 = part * spw, j1 = min(j0 + spw, n_steps);
    if (j0 >= j1) return;
    const int64_t row0 = p.seq_off ? p.seq_off[s] : (int64_t)s * (RING ? p.ring_cap : p.kv_len);
    const int qoff0 = len - p.T;  // position of token 0
    const uint32_t stride_b = (uint32_t)p.row_stride * 2;
    // (ring caches: key j sits in row j % ring_cap)
    const uint32_t nrec = (uint32_t)(RING ? p.ring_cap : len) * stride_b;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.k + row0 * p.row_stride + (size_t)kvh * HD), (short)0, (int)nrec, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.v + row0 * p.row_stride + (size_t)kvh * HD), (short)0, (int)nrec, kBufferFlags);
    const uint32_t qtok_b = (uint32_t)p.q_tok * 2;  // bytes between consecutive tokens' queries
    auto q_rsrc = [&](int j) {
        const int t0 = j * TBK, t1 = min(t0 + TBK, p.T);
        return __builtin_amdgcn_make_buffer_rsrc(
            (void*)(static_cast<const uint16_t*>(p.q) + ((size_t)s * p.T + t0) * p.q_tok), (short)0,
            (int)((uint32_t)(t1 - t0) * qtok_b), kBufferFlags);
    };
    // chunks [first, last] of block j: keys a row of the block sees
    auto chunk_lo = [&](int j) { return max(0, qoff0 + j * TBK + 1 - p.window) >> 5; };
    auto chunk_hi = [&](int j) { return (qoff0 + min(j * TBK + TBK, p.T) - 1) >> 5; };
    auto slot = [](int c) { return c % NCH; };
    // chunk c into its ring slot: waves 0-3 bring its K, 4-7 its V (one
    // 16-byte piece per lane; the lane loads the logical piece its slot holds)
    auto load_chunk = [&](int c, bool tracked) {
        const int lane = fresh_lane();
        const bool is_v = wave >= 4;
        const int q = 64 * (wave & 3) + lane, key = q / PPR, phys = q % PPR;
        const int piece = is_v ? phys ^ ((key & 3) << 1) : phys ^ (key & 7);
        const int krow = RING ? (32 * c + key) % p.ring_cap : 32 * c + key;
        const uint32_t off = (uint32_t)krow * stride_b + 16 * piece;
        char* const dst = (is_v ? vring : kring) + slot(c) * CHB + 1024 * (wave & 3);
        if (tracked) lds_dma16(is_v ? rv : rk, off, dst);
        else lds_dma16_untracked(is_v ? rv : rk, off, dst);
    };
    // the wave's query rows of block j into its staging area: instruction i
    // brings token 8 wave + i (its 8 heads, 1 KB), row 8 i + lane / 8, the
    // row's 16-byte pieces swizzled by its low 3 bits
    auto load_q_stage = [&](int j) {
        const __amdgpu_buffer_rsrc_t rq = q_rsrc(j);
        const int lane = fresh_lane(), hr = lane / PPR, phys = lane % PPR;
#pragma unroll
        for (int i = 0; i < RT * 32 / HPK; ++i) {
            const int row = HPK * i + hr;
            const uint32_t off = (uint32_t)(HPK * wave + i) * qtok_b + (uint32_t)((kvh * HPK + hr) * HD) * 2 +
                                 16 * (phys ^ (row & 7));
            lds_dma16_untracked<kSlideLoadAux == 2>(rq, off, stage + 1024 * i);
        }
    };

    static_assert(CHB / 16 <= 64 * NW, "one zero store per thread");
    if (tid < CHB / 16) *reinterpret_cast<u32x4*>(vzero + 16 * tid) = u32x4{0, 0, 0, 0};
    // first block's chunks, then its queries straight into registers
    for (int c = chunk_lo(j0); c <= chunk_hi(j0); ++c) load_chunk(c, true);
    half8 qb[RT][KS];
    {
        const __amdgpu_buffer_rsrc_t rq = q_rsrc(j0);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int r = (wave * RT + rt) * 32 + c32;
            const uint32_t qoff = (uint32_t)(r / HPK) * qtok_b + (uint32_t)((kvh * HPK + r % HPK) * HD + 8 * h2) * 2;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                qb[rt][ks] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + 32 * ks, 0, kSlideLoadAux));
        }
    }
    float sk[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = (wave * RT + rt) * 32 + c32;
        sk[rt] = p.sinks ? p.sinks[kvh * HPK + r % HPK] * kLog2e : 0.f;
    }

    float m[RT], l[RT];
    float16v o[DT][RT];
    int posr[RT], lor[RT];
    bool valid[RT];
    int c0 = 0;  // the wave's first chunk of the current block
    const half2 one2 = {(_Float16)1.f, (_Float16)1.f};
    constexpr float kSumLimit = 16384.f;

    // the wave's normalised rows of block j -> staging area -> whole rows out
    auto store_out = [&](int j) {
        const int t0 = j * TBK, t1 = min(t0 + TBK, p.T);
        const int lane = fresh_lane(), c32 = lane & 31, h2 = lane >> 5;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float inv = 1.f / half_sum(l[rt]);
            const int rl = rt * 32 + c32;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const half4 hv = {(_Float16)(o[dt][rt][4 * i4] * inv), (_Float16)(o[dt][rt][4 * i4 + 1] * inv),
                                      (_Float16)(o[dt][rt][4 * i4 + 2] * inv), (_Float16)(o[dt][rt][4 * i4 + 3] * inv)};
                    const int pc = 4 * dt + i4;
                    *reinterpret_cast<half4*>(stage + rl * (HD * 2) + ((pc ^ (rl % PPR)) << 4) + 8 * h2) = hv;
                }
        }
        // every row read back first, then the stores through a buffer
        // resource over the block's output rows (rows past the prompt fall
        // outside it and are dropped: no branch per store)
        constexpr int RPI = 64 / PPR;
        constexpr int NST = RT * 32 / RPI;
        const int pc = lane % PPR;
        u32x4 val[NST];
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            const int rl = k * RPI + lane / PPR;
            val[k] = *reinterpret_cast<const u32x4*>(stage + rl * (HD * 2) + ((pc ^ (rl % PPR)) << 4));
        }
        const uint32_t otok_b = (uint32_t)p.o_tok * 2;
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(static_cast<uint16_t*>(p.out) + ((size_t)s * p.T + t0) * p.o_tok), (short)0,
            (int)((uint32_t)(t1 - t0) * otok_b), kBufferFlags);
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            const int r = wave * RT * 32 + k * RPI + lane / PPR;  // token r / HPK of the block, head r % HPK
            const uint32_t off = (uint32_t)(r / HPK) * otok_b + (uint32_t)((kvh * HPK + r % HPK) * HD + 8 * pc) * 2;
            __builtin_amdgcn_raw_buffer_store_b128(val[k], ro, off, 0, kSlideStoreAux);
        }
    };

    // S^T of chunk c (wave-local index) into sc
    auto qk = [&](int c, float16v (&sc)[RT]) {
        const char* kt = kring + slot(c0 + c) * CHB;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sc[rt] = float16v{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const half8 ka = *reinterpret_cast<const half8*>(kt + k_slot<HD>(c32, 2 * ks + h2));
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) sc[rt] = mfma32(ka, qb[rt][ks], sc[rt]);
        }
    };
    auto pv = [&](int c, const half8 (&pb)[2][RT]) {
        const char* vt = vring + slot(c0 + c) * CHB;
        const int G = lane >> 4, r4 = (lane & 15) >> 2, q4 = lane & 3;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            half8 va[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int key = 16 * w + 4 * h2 + r4, dim = 32 * dt + 16 * (G & 1) + 4 * q4;
                const _Float16* a0 = reinterpret_cast<const _Float16*>(vt + v_slot<HD>(key, dim >> 3) + ((dim & 7) << 1));
                const _Float16* a1 = reinterpret_cast<const _Float16*>(vt + v_slot<HD>(key + 8, dim >> 3) + ((dim & 7) << 1));
                va[dt] = cat8(lds_read_tr(a0), lds_read_tr(a1));
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) o[dt][rt] = mfma32(va[dt], pb[w][rt], o[dt][rt]);
        }
    };

    float16v s_a[RT], s_b[RT];
    half8 p_a[2][RT], p_b[2][RT];
    int wpf = 0, wlo_last = 0;  // the wave's first row position and last row's window start

    // one chunk: prefill_kernel's step with ring addresses
    auto step = [&](int c, float16v (&s_cur)[RT], float16v (&s_nxt)[RT], const half8 (&p_prv)[2][RT],
                    half8 (&p_cur)[2][RT]) {
        const int kb = 32 * (c0 + c);
        if (kb + 31 > wpf || kb < wlo_last) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kb + 8 * (i / 4) + 4 * h2 + (i % 4);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    if (key < lor[rt] || key > posr[rt]) s_cur[rt][i] = -INFINITY;
            }
        }
        constexpr int NOPD = KS + 2 * DT;
        half8 opd[NOPD];
        const char* const kt_c = kring + slot(c0 + c + 1) * CHB;  // (past the last chunk: discarded)
        const char* const vt_c = c == 0 ? vzero : vring + slot(c0 + c - 1) * CHB;
        auto read_opd = [&](int r) {
            if (r < KS) {
                opd[r] = *reinterpret_cast<const half8*>(kt_c + k_slot<HD>(c32, 2 * r + h2));
            } else {
                const int w = (r - KS) / DT, dt = (r - KS) % DT;
                const int G = lane >> 4, r4 = (lane & 15) >> 2, q4 = lane & 3;
                const int key = 16 * w + 4 * h2 + r4, dim = 32 * dt + 16 * (G & 1) + 4 * q4;
                const _Float16* a0 = reinterpret_cast<const _Float16*>(vt_c + v_slot<HD>(key, dim >> 3) + ((dim & 7) << 1));
                const _Float16* a1 = reinterpret_cast<const _Float16*>(vt_c + v_slot<HD>(key + 8, dim >> 3) + ((dim & 7) << 1));
                opd[r] = cat8(lds_read_tr(a0), lds_read_tr(a1));
            }
        };
        read_opd(0);
        read_opd(1);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) s_nxt[rt] = float16v{};
        constexpr int NM = KS * RT + 2 * DT * RT;
        constexpr int NS = 16 * RT;
        constexpr int NP = NS / 2;
        static_assert(NS % NM == 0, "whole scores per MFMA slot");
        constexpr int S = NS / NM;
        float ms[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) ms[rt] = m[rt] == -INFINITY ? 0.f : m[rt];
        float acc[RT][2];
        float e[NS];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt][0] = acc[rt][1] = 0.f;
        auto op_fma = [&](int i) {
            if (i < NS) s_cur[i / 16][i % 16] = __builtin_fmaf(s_cur[i / 16][i % 16], p.qscale, -ms[i / 16]);
        };
        auto op_exp = [&](int i) {
            if (i < NS) e[i] = fast_exp2(s_cur[i / 16][i % 16]);
        };
        auto op_pack = [&](int k) {
            const int rt = k / 8, i = 2 * (k % 8);
            p_cur[i / 8][rt][i % 8] = (_Float16)e[2 * k];
            p_cur[i / 8][rt][i % 8 + 1] = (_Float16)e[2 * k + 1];
        };
        auto op_dot = [&](int k) {
            const int rt = k / 8, i = 2 * (k % 8);
            acc[rt][k & 1] = __builtin_amdgcn_fdot2(half2{p_cur[i / 8][rt][i % 8], p_cur[i / 8][rt][i % 8 + 1]}, one2,
                                                    acc[rt][k & 1], false);
        };
        auto packable = [](int u) { return u < 0 ? 0 : (S * (u + 1)) / 2; };
#pragma unroll
        for (int j = 0; j < S; ++j) op_fma(j);
#pragma unroll
        for (int t = 0; t < NM; ++t) {
            const int r = t / RT;
            if (t % RT == 0 && r + 2 < NOPD) read_opd(r + 2);
            if (t < KS * RT) {
                const int rt = t % RT;
                s_nxt[rt] = mfma32(opd[r], qb[rt][r], s_nxt[rt]);
            } else {
                const int j = t - KS * RT, w = j / (DT * RT), dt = (j / RT) % DT, rt = j % RT;
                o[dt][rt] = mfma32(opd[r], p_prv[w][rt], o[dt][rt]);
            }
#pragma unroll
            for (int k = packable(t - 3); k < packable(t - 2); ++k) op_dot(k);
#pragma unroll
            for (int k = packable(t - 2); k < packable(t - 1); ++k) op_pack(k);
#pragma unroll
            for (int j = 0; j < S; ++j) op_exp(S * t + j);
#pragma unroll
            for (int j = 0; j < S; ++j) op_fma(S * (t + 1) + j);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int k = packable(NM - 2); k < NP; ++k) op_pack(k);
#pragma unroll
        for (int k = packable(NM - 3); k < NP; ++k) op_dot(k);
        float ls[RT];
        bool bad = false;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            ls[rt] = acc[rt][0] + acc[rt][1];
            bad |= !(ls[rt] <= kSumLimit) || m[rt] == -INFINITY;
        }
#ifdef PELICA_PTRACE
        n_exact += __builtin_amdgcn_ballot_w64(bad) != 0;
#endif
        if (__builtin_amdgcn_ballot_w64(bad)) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                float x = -INFINITY;
#pragma unroll
                for (int i = 0; i < 16; ++i) x = fmaxf(x, s_cur[rt][i]);
                const float mn = fmaxf(m[rt], half_max(x) + ms[rt]);
                if (mn > m[rt]) {
                    const float cf = fast_exp2(m[rt] - mn);
                    l[rt] *= cf;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) o[dt][rt] *= cf;
                    m[rt] = mn;
                }
                const float shift = ms[rt] - (m[rt] == -INFINITY ? 0.f : m[rt]);
                float a = 0.f;
#pragma unroll
                for (int w = 0; w < 2; ++w)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        p_cur[w][rt][j] = (_Float16)fast_exp2(s_cur[rt][8 * w + j] + shift);
                        a += (float)p_cur[w][rt][j];
                    }
                ls[rt] = a;
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) l[rt] += ls[rt];
    };

    for (int j = j0; j < j1; ++j) {
        const int t0 = j * TBK, t1 = min(t0 + TBK, p.T);

        // The loads of block j (chunks and, after the first block, queries)
        // have landed, and every wave is done with block j-1's chunks.
#ifdef PELICA_PTRACE
        const unsigned ta = cyc();
        __builtin_amdgcn_s_waitcnt(0x0F70);
        const unsigned tb2 = cyc();
        __syncthreads();
        t_wait += tb2 - ta;
        t_bar += cyc() - tb2;
        if (lane == 0 && j == j0 + 1) g_ptrace[wid * 16 + 12] = rtime();
#else
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
#endif
        if (j > j0) {
            // block j's queries from the staging area, then block j-1's
            // output through it (a wave's LDS accesses complete in order)
            const int lane = fresh_lane(), c32 = lane & 31, h2 = lane >> 5;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int rl = rt * 32 + c32;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    qb[rt][ks] = *reinterpret_cast<const half8*>(stage + rl * (HD * 2) + (((2 * ks + h2) ^ (rl & 7)) << 4));
            }
#ifdef PELICA_PTRACE
            if (lane == 0 && j == j0 + 1) g_ptrace[wid * 16 + 13] = rtime();
#endif
            store_out(j - 1);
#ifdef PELICA_PTRACE
            if (lane == 0 && j == j0 + 1) g_ptrace[wid * 16 + 14] = rtime();
#endif
        }
        // block j+1's new chunks and queries, in flight while j is computed
        if (j + 1 < j1) {
            for (int c = chunk_hi(j) + 1; c <= chunk_hi(j + 1); ++c) load_chunk(c, false);
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the staging area's reads are done
            load_q_stage(j + 1);
        }
        // this wave's rows of block j: tokens t0 + 8 wave .. + 7
        const int tw0 = t0 + RT * 32 / HPK * wave;
        const int tw1 = min(tw0 + RT * 32 / HPK, t1);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int r = (wave * RT + rt) * 32 + c32;
            const int t = t0 + r / HPK;
            valid[rt] = t < t1;
            posr[rt] = valid[rt] ? qoff0 + t : -1;
            lor[rt] = (posr[rt] + 1 > p.window) ? posr[rt] + 1 - p.window : 0;
            m[rt] = valid[rt] ? (p.sinks ? sk[rt] : -INFINITY) : 0.f;
            l[rt] = (valid[rt] && p.sinks && h2 == 0) ? 1.f : 0.f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt][rt] = float16v{};
        }
        if (tw0 >= tw1) continue;  // (no rows: past the prompt)
        wpf = qoff0 + tw0;
        const int wpl = qoff0 + tw1 - 1;
        wlo_last = max(0, wpl + 1 - p.window);
        c0 = max(0, wpf + 1 - p.window) >> 5;
        const int nch = (wpl >> 5) - c0 + 1;
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) p_b[w][rt] = half8{0, 0, 0, 0, 0, 0, 0, 0};
#ifdef PELICA_PTRACE
        const unsigned tc0 = cyc();
        {
            const unsigned long long r0 = rtime();
            if (j == j0) rt_first = r0;
            if (lane == 0 && j - j0 < 3) g_ptrace[wid * 16 + 8 + 2 * (j - j0)] = r0;
        }
        n_ch_all += nch;
#endif
        qk(0, s_a);
        // every chunk unrolled (a wave sees at most 6: 8 tokens under a
        // window of up to 130 keys)
        step(0, s_a, s_b, p_b, p_a);
        if (nch > 1) step(1, s_b, s_a, p_a, p_b);
        if (nch > 2) step(2, s_a, s_b, p_b, p_a);
        if (nch > 3) step(3, s_b, s_a, p_a, p_b);
        if (nch > 4) step(4, s_a, s_b, p_b, p_a);
        if (nch > 5) step(5, s_b, s_a, p_a, p_b);
        if (nch & 1) pv(nch - 1, p_a);
        else pv(nch - 1, p_b);
#ifdef PELICA_PTRACE
        t_comp += cyc() - tc0;
        rt_last = rtime();
        if (lane == 0 && j - j0 < 3) g_ptrace[wid * 16 + 9 + 2 * (j - j0)] = rt_last;
#endif
    }
    store_out(j1 - 1);
#ifdef PELICA_PTRACE
    if (lane == 0) {
        g_ptrace[wid * 16 + 0] = t_comp;
        g_ptrace[wid * 16 + 1] = t_wait;
        g_ptrace[wid * 16 + 2] = t_bar;
        g_ptrace[wid * 16 + 3] = (unsigned long long)n_exact << 32 | n_ch_all;
        g_ptrace[wid * 16 + 4] = rt_entry;
        g_ptrace[wid * 16 + 5] = rt_first;
        g_ptrace[wid * 16 + 6] = rt_last;
        g_ptrace[wid * 16 + 7] = rtime();
        g_ptrace[wid * 16 + 15] = 1;
    }
#endif
}

// 64-key tiles a token block of TB tokens can need under a window: keys
// [pos_first + 1 - window, pos_last] from a 32-aligned start (0: no bound)
static int window_tiles(int window, int TB) {
    if (window <= 0) return 0;
    const int chunks = (TB - 1 + window - 1 + 31) / 32 + 1;
    return (chunks + 1) / 2;
}

template <int HD, int RT, int NW, bool F32>
static hipError_t launch_nw(const PrefillParams& p, hipStream_t st) {
    constexpr int ROWS = NW * RT * 32;
    if (p.hpk > ROWS) return hipErrorNotSupported;
    const int TB = ROWS / p.hpk;
    const int n_tb = (p.T + TB - 1) / TB;
    const long long nblk = (long long)n_tb * p.n_kv * p.n_seq;
    if (nblk > 0x7fffffff) return hipErrorNotSupported;
    ProfScope ps(kProfPrefill, st);
    const dim3 grid((unsigned)nblk), block(64 * NW);
    // head dim 64: short windows keep all their K/V tiles in LDS (<= 3 of
    // each: 56 KB, two 4-wave workgroups per CU)
    const int wt = window_tiles(p.window, TB);
    const bool res = HD == 64 && !p.state && wt > 0 && wt <= 3;
    if constexpr (HD == 64 && NW == 4) {
        if (res) {
            if (p.ring_cap) hipLaunchKernelGGL((prefill_kernel<HD, RT, true, false, NW, 3, F32>), grid, block, 0, st, p, n_tb, TB);
            else hipLaunchKernelGGL((prefill_kernel<HD, RT, false, false, NW, 3, F32>), grid, block, 0, st, p, n_tb, TB);
            return hipGetLastError();
        }
    }
    if (p.state)
        hipLaunchKernelGGL((prefill_kernel<HD, RT, false, true, NW, 0, F32>), grid, block, 0, st, p, n_tb, TB);
    else if (p.ring_cap)
        hipLaunchKernelGGL((prefill_kernel<HD, RT, true, false, NW, 0, F32>), grid, block, 0, st, p, n_tb, TB);
    else
        hipLaunchKernelGGL((prefill_kernel<HD, RT, false, false, NW, 0, F32>), grid, block, 0, st, p, n_tb, TB);
    return hipGetLastError();
}

// Workgroup size: 8 waves (2 per SIMD from one workgroup: each K/V tile in
// LDS serves twice the rows; the 4096-token gpt-oss causal prefill ~2 %
// faster) unless a short window makes the larger token block mostly masked
// (window 128: 4 waves, 25 % faster than 8).
// ring slots of the sliding-window kernel: the chunks of two consecutive
// 64-token blocks, (126 + window) / 32 + 2, fit for windows up to 130
constexpr int kSlideChunks = 10;

static int prefill_cus() {
    static const int n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        return cus;
    }();
    return n;
}

// the sliding-window kernel's shapes: head dim 64, 8 heads per kv head,
// whole-prompt launches, a window its chunk ring holds
static bool slide_fits(const PrefillParams& p) {
    return p.hd == 64 && p.hpk == 8 && !p.state && p.window > 0 &&
           (126 + p.window) / 32 + 2 <= kSlideChunks;
}

static hipError_t launch_slide(const PrefillParams& p, hipStream_t st) {
    const int n_steps = (p.T + 63) / 64;
    const long long total = (long long)n_steps * p.n_kv * p.n_seq;
    const int spw = (int)std::max(1LL, (total + prefill_cus() - 1) / prefill_cus());
    const int n_parts = (n_steps + spw - 1) / spw;
    const long long nblk = (long long)n_parts * p.n_kv * p.n_seq;
    if (nblk > 0x7fffffff) return hipErrorNotSupported;
    ProfScope ps(kProfPrefill, st);
    if (p.ring_cap)
        hipLaunchKernelGGL((prefill_slide_kernel<kSlideChunks, true>), dim3((unsigned)nblk), dim3(512), 0, st, p, n_parts,
                           spw);
    else
        hipLaunchKernelGGL((prefill_slide_kernel<kSlideChunks, false>), dim3((unsigned)nblk), dim3(512), 0, st, p,
                           n_parts, spw);
    return hipGetLastError();
}

template <int HD, int RT, bool F32>
static hipError_t launch(const PrefillParams& p, hipStream_t st) {
    if (HD == 64 && RT == 2 && !F32 && slide_fits(p)) return launch_slide(p, st);
    if (p.window > 0 && p.window <= 1024) return launch_nw<HD, RT, 4, F32>(p, st);
    return launch_nw<HD, RT, 8, F32>(p, st);
}

#ifdef PELICA_PTRACE
extern "C" int pelica_attn_debug_ptrace(void* dst, size_t bytes) {
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_ptrace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

hipError_t launch_prefill(const PrefillParams& p, hipStream_t st) {
    if (p.f32) {
        if (p.hd == 64) return launch<64, 2, true>(p, st);
        if (p.hd == 128) return launch<128, 1, true>(p, st);
    } else {
        if (p.hd == 64) return launch<64, 2, false>(p, st);
        if (p.hd == 128) return launch<128, 1, false>(p, st);
    }
    return hipErrorNotSupported;
}

}  // namespace pelica
