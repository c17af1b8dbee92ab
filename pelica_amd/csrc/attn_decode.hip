// Split-K flash-decode for gfx950: f32 queries, f16 KV cache, f32 output.
//
// Work split.  A workgroup of NW waves owns (sequence s, wg_heads
// consecutive kv heads, row group, key split): wave w serves kv head
// w % wg_heads and takes every (NW / wg_heads)-th 64-key block of the split.
// The waves of the different heads walk the same keys side by side, so each
// cache row (all kv heads of a position, adjacent in memory) is fetched by
// one workgroup at one time — on MI355X, spreading a row's head slices over
// workgroups that reach it at different times costs ~25% of HBM throughput.
// All query rows that share kv head g — the GQA group times the pass's
// tokens (drafts) — ride in the same wave, so every K/V byte is read from
// HBM once.  Rows sit in the MFMA's 16-wide n dimension.
//
// Per 64-key block (one block in flight per wave):
//   K and V go from HBM straight into the wave's own K and V LDS buffers
//      (buffer_load ... lds, streaming `nt`) in whole 128-byte lines; each
//      lane loads the piece that an XOR swizzle puts in its LDS slot, which
//      keeps the operand reads below bank-conflict free.  K's loads are
//      issued before V's; the next block's K (V) loads go out as soon as
//      this block's K (V) reads are done;
//   S^T[key][row] = K Q^T on v_mfma_f32_16x16x32_f16, K read from LDS in
//      the A-operand layout (ds_read_b128).  Q is split into f16 hi + lo
//      parts so the scores keep ~fp32 accuracy: with <= 8 rows both parts
//      share one MFMA (hi in columns 0-7, lo in 8-15, summed across lanes
//      l, l^8), otherwise they take two;
//   online softmax in base 2 (log2(e) folded into the query scale); block
//      max and sums over the four 16-lane groups with permlane swaps; masks
//      only on blocks that cross a row's key range;
//   O^T = V^T P^T with V read by the transposing ds_read_b64_tr_b16 as the
//      A operand and P (hi + lo, packed like Q) as the B operand straight
//      from the score registers (its key order matches the A operand's).
// The wave states of each head merge without a workgroup barrier: each wave
// leaves its state in its LDS buffer and counts itself in on the head's LDS
// counter, and the last to arrive merges them in wave order into one partial
// (max, sum, O) per row and split.  A combine kernel (one 256-thread
// workgroup per query row, or one wave per row when rows have few splits)
// merges the splits in key order with the head's sink; a single split
// writes the output directly.  (In-kernel combines were
// measured slower on MI355X: the last workgroup alone reading every partial,
// a grid barrier on one device-scope counter — its atomics serialise — and
// per-workgroup flags that every workgroup polls.)
//
// Ragged batches (no window, no ring) run stream-K instead of one grid of
// equal key splits: with a split grid the workgroups of the longest
// sequences set the time (32 sequences of 512-16K keys: 180 busy
// workgroups, then a long tail).  A
// fixed grid of about one workgroup per CU cuts the batch's list of 64-key
// blocks into equal contiguous ranges; a range may end inside one sequence's
// segment and continue into the next, and each such piece is a split with
// its own slot.  Piece starts are charged in the list (SkLayout) because a
// piece refills the load pipeline.
//
// Reference semantics: src/moe_kernels.rs:482-617 (attn_dec, merge_dec),
// src/oss_batch.rs:172-251 (ATTN_T: window, ring, sink), :253-425 (attn_s +
// ATTN_M: split partials, sink in max and denominator).
#include <algorithm>

#include "attn_decode.hpp"
#include "attn_prof.hpp"

namespace pelica {

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

// waves per SIMD the decode kernel is compiled for (register budget 512/n)
template <int HD, int RT, int NW>
constexpr int kDecodeOcc = NW == 8 ? 2 : (NW == 4 && HD == 64 && RT <= 2) ? 2 : 1;


// word 3 of a gfx9 buffer resource: 32-bit data format, raw addressing
constexpr int kBufferFlags = 0x00020000;
// cache policy of write-through stores (sc1): partials that another XCD's
// combine workgroup reads
constexpr int kPartWriteThrough = 16;

// Visible keys of one query: [lo, pos].
struct KeyRange {
    int lo, pos;
};

// Keys query token t of a sequence of len keys sees: [lo, pos] under the
// window, clipped to the call's key range [kr_lo, kr_hi) (the whole cache
// unless the call covers one range of positions)
__device__ __forceinline__ KeyRange key_range(const DecodeParams& p, int len, int t) {
    const int pos = len - p.T + t;
    const int lo = (p.window > 0 && pos + 1 > p.window) ? pos + 1 - p.window : 0;
    return KeyRange{max(lo, p.kr_lo), min(pos, p.kr_hi - 1)};
}

// LDS byte offset of 16-byte piece p of key row k in a V block: rows of HD
// halfs, pieces XOR-swizzled so the transposed reads of 4 consecutive keys
// hit distinct banks.
template <int HD>
__device__ __forceinline__ int v_slot(int k, int p) {
    return k * (HD * 2) + ((p ^ ((k & 3) << 1)) << 4);
}

template <int HD>
__device__ __forceinline__ const _Float16* v_elem(const _Float16* base, int k, int d) {
    return reinterpret_cast<const _Float16*>(reinterpret_cast<const char*>(base) + v_slot<HD>(k, d >> 3) +
                                             ((d & 7) << 1));
}

// One merge_dec partial slot {M (natural log), L, O[hd]} (8-byte aligned):
// this thread's 4 dims at d, and the (max, sum) pair from the d == 0 thread.
__device__ __forceinline__ void store_part(float* slot, int d, float m2, float l, const float4v& o) {
    if (d == 0) *reinterpret_cast<float2*>(slot) = make_float2(m2 == -INFINITY ? -3.0e38f : m2 * kLn2, l);
    *reinterpret_cast<float2*>(slot + 2 + d) = make_float2(o[0], o[1]);
    *reinterpret_cast<float2*>(slot + 4 + d) = make_float2(o[2], o[3]);
}

// Build-time instrumentation (off by default; -DPELICA_DTRACE): lane 0 of
// every split-kernel wave stores s_memrealtime stamps (100 MHz) at start,
// first K block landed, V blocks 0 and 1 landed, loop end, merge hand-off
// (the merging wave: merge done) and end, plus its XCC/hardware id, into
// g_dtrace[wave * 8 + k] (the
// first 8192 waves of the grid);
// pelica_attn_debug_trace() copies the array out after a call.
#ifdef PELICA_DTRACE
__device__ unsigned long long g_dtrace[1 << 16];
#define DTRACE(k) do { \
    const size_t i_ = ((((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * NW + wave) * 8 + (k); \
    if (lane == 0 && i_ < (1u << 16)) \
        g_dtrace[i_] = (k) == 7 ? ((unsigned long long)__builtin_amdgcn_s_getreg(6164) << 32 | __builtin_amdgcn_s_getreg(63492)) \
                                : __builtin_amdgcn_s_memrealtime(); \
} while (0)
#else
#define DTRACE(k) do {} while (0)
#endif

// K blocks in LDS: 16-byte piece p of key row k sits at slot p ^ k_swz(k), so
// the 16 keys that one ds_read_b128 of the QK^T A operand touches (same
// piece) fall in distinct banks, and the 8 (hd 64) or 4 (hd 128) keys of one
// full-line global load keep a per-lane swizzle that differs between loads
// only by a constant (k_swz_j).
template <int HD>
__device__ __forceinline__ int k_swz(int k) {
    return HD == 64 ? (((k >> 1) ^ ((k & 1) << 2)) & 7) : (k & 15);
}
// k_swz(KPL * j + k0) == k_swz(k0) ^ k_swz_j(j) for k0 < KPL (KPL = keys per
// 64-lane load: 8 for hd 64, 4 for hd 128)
template <int HD>
__device__ constexpr int k_swz_j(int j) {
    return HD == 64 ? 4 * (j & 1) : (4 * j) & 15;
}

// 16 bytes per lane from a buffer resource straight into LDS at lds + 16 *
// lane, with the K/V stream's cache policy; `tracked` false: issued so the
// compiler does not track it (loads inside the block loop, whose waits are
// counted by hand; lds_dma16_untracked)
__device__ __forceinline__ void kv_dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, char* lds, bool tracked) {
    if (tracked) lds_dma16<true>(rsrc, voffset, lds);
    else lds_dma16_untracked<true>(rsrc, voffset, lds);
}

// s_waitcnt vmcnt(N), the other counters left alone (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
    __asm__ volatile("" ::: "memory");
}
// s_waitcnt lgkmcnt(0)
__device__ __forceinline__ void wait_lgkm0() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __asm__ volatile("" ::: "memory");
}

// the value of lane l ^ 8 (within each 16-lane row)
__device__ __forceinline__ float ror8(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
}

// Stream-K layout of a ragged batch (no window, no ring): the segments (a
// sequence's blocks of one row group and kv head), sequence-major, form one
// list in which segment i takes p.sk_restart positions for its start-up (a
// piece restarts the load pipeline: ~8-11 blocks' time) and then its
// 64-key blocks.  The list is cut into g_eff equal contiguous ranges, one
// per workgroup (at least p.sk_minb positions each), so a workgroup whose
// range crosses a segment start gets correspondingly fewer blocks.  Each
// piece of a segment is one split (slot = its index among the segment's
// pieces).
// List positions are 32-bit: the planner takes stream-K only for lists under
// 2^31 positions (64-bit divisions and their register pressure cost the
// kernel's prologue microseconds before its first load).
struct SkLayout {
    int total;          // positions in the list
    int g_eff, q, rem;  // workgroups used; range of w: q blocks (+1 if w < rem)
    __device__ int start(int w) const { return w * q + min(w, rem); }
    // the workgroup whose range holds block x
    __device__ int owner(int x) const {
        const int big = rem * (q + 1);
        return x < big ? x / (q + 1) : rem + (x - big) / q;
    }
};

__device__ __forceinline__ int uniform32(int x) { return __builtin_amdgcn_readfirstlane(x); }

// blocks of a sequence of len keys in the stream-K list (0 for a skipped sequence)
__device__ __forceinline__ int sk_blocks_of(const DecodeParams& p, int len) {
    return (len < p.T || len <= 0) ? 0 : (len + 63) / 64;
}
// list positions of one segment of a sequence of len keys (start-up + blocks, or 0)
__device__ __forceinline__ int sk_span_of(const DecodeParams& p, int len) {
    const int nb = sk_blocks_of(p, len);
    return nb ? nb + p.sk_restart : 0;
}

// The batch's sequence tables as the stream-K driver reads them: for up to
// 64 sequences lane i holds sequence i's key count and first cache row,
// loaded once (one memory round trip for both) and read with readlane
// afterwards; larger batches read the tables from memory each time.
struct SeqTables {
    bool cached;
    int len;         // this lane's sequence's keys (cached)
    long long off;   // its first cache row (cached)
    __device__ int keys(const DecodeParams& p, int s) const {  // s uniform
        return cached ? __builtin_amdgcn_readlane(len, s) : seq_keys(p.seq_len, s, p.kv_len);
    }
    __device__ int keys_lane(const DecodeParams& p, int s) const {  // s = base + lane
        return cached ? len : seq_keys(p.seq_len, s, p.kv_len);
    }
    __device__ long long row0(const DecodeParams& p, int s) const {  // s uniform
        if (!cached) return p.seq_off ? p.seq_off[s] : (long long)s * p.kv_len;
        const unsigned lo = __builtin_amdgcn_readlane((unsigned)off, s);
        const unsigned hi = __builtin_amdgcn_readlane((unsigned)((unsigned long long)off >> 32), s);
        return (long long)((unsigned long long)hi << 32 | lo);
    }
};

__device__ __forceinline__ SeqTables seq_tables(const DecodeParams& p) {
    const int lane = threadIdx.x & 63;
    SeqTables t{p.n_seq <= 64, 0, 0};
    if (t.cached && lane < p.n_seq) {
        t.len = seq_keys(p.seq_len, lane, p.kv_len);
        t.off = p.seq_off ? p.seq_off[lane] : (long long)lane * p.kv_len;
    }
    return t;
}

// the layout, computed by every lane of the calling wave (uniform result)
__device__ SkLayout sk_layout(const DecodeParams& p, int gy, const SeqTables& tb) {
    const int lane = threadIdx.x & 63;
    int tot = 0;
    for (int base = 0; base < p.n_seq; base += 64) {
        int x = base + lane < p.n_seq ? sk_span_of(p, tb.keys_lane(p, base + lane)) : 0;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
        tot += x;
    }
    SkLayout L;
    L.total = uniform32(tot * gy);
    L.g_eff = uniform32(max(1, min(p.sk_grid, L.total / p.sk_minb)));
    L.q = uniform32(L.total / L.g_eff);
    L.rem = uniform32(L.total % L.g_eff);
    return L;
}

template <int HD, int RT, int NW, int H, bool SK>
constexpr int kDecodeOccK = SK ? ((HD == 64 && RT == 1) ? kDecodeOcc<HD, RT, NW> : 1) : kDecodeOcc<HD, RT, NW>;

template <int HD, int RT, int NW, int H, bool RING, bool PK, bool SK>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(kDecodeOccK<HD, RT, NW, H, SK>, 8))) void decode_kernel(DecodeParams p) {
    static_assert(!SK || (H == 1 && !RING), "stream-K: one kv head per workgroup, linear caches");
    static_assert(!PK || RT == 1, "packed hi/lo columns need one row tile");
    constexpr int DS = HD / 32;   // 32-dim k-steps of the QK^T MFMA
    constexpr int DT = HD / 16;   // 16-dim output tiles
    constexpr int VPL = HD / 8;   // 16-byte pieces per lane per block, each of K and V
    constexpr int ROWS = RT * 16;
    constexpr bool EARLY_V = HD == 64 && !SK;
    // one-wave workgroups (small head-dim-128 calls) store their split
    // partials write-through: OLMoE 2K / Qwen3 8K decode 9.85 -> 9.71 /
    // 10.32 -> 9.85 us a call (the gpt-oss 32K call and ragged verify
    // batches were even and 2 % slower that way)
    constexpr bool PART_WT = NW == 1;
    // f16 parts (hi + lo) of Q and P: packed (PK: hi in columns 0-7, lo in
    // 8-15, one MFMA), or separate passes: NP of Q, NPP of P
    constexpr int NP = PK ? 1 : 2;
    constexpr int NPP = PK ? 1 : 2;
    constexpr int BUF = 64 * HD * 2;                   // bytes of one 64-key K or V block
    constexpr int STATE = DT * RT * 64 * 16 + RT * 64 * 8;  // bytes of one wave's (O, m, l)
    // LDS per wave: a K and a V block buffer, filled straight from HBM;
    // after the last block, the wave's state
    constexpr int WSLOT = 2 * BUF > STATE ? 2 * BUF : STATE;
    constexpr int SMEM = WSLOT * NW;
    __shared__ __attribute__((aligned(16))) char smem[SMEM];
    __shared__ unsigned arrivals[H];  // waves of each head done (merge at the end)

    // wave index as a scalar: the buffer resources built from it stay in SGPRs
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
              c16 = lane & 15;
    constexpr int W = NW / H;                   // waves per head
    const int hl = wave % H, wsub = wave / H;   // this wave's head (local) and block phase
    DTRACE(0);
    DTRACE(7);
    const int hgroups = p.n_kv / H;

    // One split: keys [kbeg, kend) of sequence s, row group and kv heads of
    // by, written to slot `slot` (single: the only split of its rows, which
    // then writes the output itself).  Uniform over the workgroup.
    auto split = [&](const int s, const int by, const int len, const int64_t row0, const int kbeg, const int kend,
                     const int slot, const bool single) {
    const int kvh = (by % hgroups) * H + hl, rg = by / hgroups;
    const int lo_min = key_range(p, len, 0).lo;
    const int rbase = rg * ROWS;

    // ---- K/V stream setup: the first block is requested before anything
    //      else, so its HBM latency overlaps the query setup ----
    // Buffer resources over this sequence's rows of kv head kvh: 32-bit
    // offsets, and loads at offsets past num_records return 0 without
    // touching memory — the tail of the last block costs no traffic.  (A
    // key range's rows start at position kr_lo: keys below it wrap to
    // offsets past num_records.)
    const uint32_t stride_b = (uint32_t)p.row_stride * 2;
    const uint32_t nrec = (RING ? (uint32_t)p.ring_cap : (uint32_t)(min(len, p.kr_hi) - p.kr_lo)) * stride_b;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.k + row0 * p.row_stride + (size_t)kvh * HD), (short)0, (int)nrec, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.v + row0 * p.row_stride + (size_t)kvh * HD), (short)0, (int)nrec, kBufferFlags);
    // Both K and V are fetched in whole 128-byte lines: load j of a block
    // gives lane l key KPL*j + l/PPR, piece l%PPR, and the lane's 16 bytes go
    // to LDS slot j*64 + l of the wave's buffer.  The lane reads the logical
    // piece that belongs in that slot under the buffer's swizzle: V
    // (v_slot) depends on the key's low two bits (the lane's own), K
    // (k_swz) on more, through a per-load constant.
    constexpr int PPR = HD / 8;         // 16-byte pieces per key row
    constexpr int KPL = 64 / PPR;       // keys per 64 lanes
    const int vk0 = lane / PPR;
    const uint32_t vcol = 16 * ((lane % PPR) ^ ((vk0 & 3) << 1));
    const uint32_t kcol0 = (lane % PPR) ^ k_swz<HD>(vk0);
    // this wave's blocks: kb = kfirst + 64 * (wsub + W * i)
    int kfirst = kbeg;
    if (lo_min > kbeg) kfirst = kbeg + ((lo_min - kbeg) & ~63);
    const int nblk_all = (kend - kfirst + 63) / 64;
    const int nb = nblk_all > wsub ? (nblk_all - wsub + W - 1) / W : 0;
    char* klds = smem + wave * WSLOT;
    char* vlds = klds + BUF;
    auto blk = [&](int i) { return kfirst + 64 * (wsub + W * i); };

    auto row_of = [&](int i, int j) -> uint32_t {
        const int kb = blk(i);
        if (i >= nb) return nrec;
        if (!RING) return (uint32_t)(kb + KPL * j + vk0 - p.kr_lo) * stride_b;
        return (uint32_t)((kb + KPL * j + vk0) % p.ring_cap) * stride_b;
    };
    // Load j of a block fills LDS slots j*64 + lane of the wave's buffer
    // (buffer_load ... lds).  K of a block is requested before its V, so
    // QK^T can start while V is still arriving.
    // (block 0's loads are tracked by the compiler; the loop's are
    // untracked, see the loop)
    auto issue_k = [&](int i, bool tracked) {
#pragma unroll
        for (int j = 0; j < VPL; ++j)
            kv_dma16(rk, row_of(i, j) + 16 * (kcol0 ^ k_swz_j<HD>(j)), klds + 1024 * j, tracked);
    };
    auto issue_v = [&](int i, bool tracked) {
#pragma unroll
        for (int j = 0; j < VPL; ++j) kv_dma16(rv, row_of(i, j) + vcol, vlds + 1024 * j, tracked);
    };
    // ---- block 0 and this lane's queries ----
    // Head dim 128: the queries are requested first (a few hundred bytes
    // per wave), then block 0 — the wait for the queries then leaves K and V
    // in flight, so QK^T starts when K lands, not once V has (measured:
    // 32-sequence draft batch 108.6 -> 105.3-107.0 us, 8K-key GQA decode
    // 11.5 -> 11.3 us; the 2K-key call's split kernel 7.75 -> 7.6 us, its
    // whole call 10.45 -> 10.6 us).
    // Head dim 64: block 0 first, the queries behind it (the next block's K
    // then goes out only once V has landed; requested earlier, it delays
    // that V and the whole stream: gpt-oss decode +0.4 us, and the 128-key
    // window call +0.7 us; with the queries first and K(1) held back until
    // V(0) has landed, gpt-oss decode is even and the window call +0.5 us).
    constexpr bool QFIRST = HD == 128;
    if (!QFIRST && nb > 0) {
        issue_k(0, true);
        issue_v(0, true);
    }
    float4v qraw[RT][DS][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = rbase + 16 * rt + (PK ? (c16 & 7) : c16);
        const int rr = r < p.R ? r : 0;
        const int t = rr / p.hpk, h = kvh * p.hpk + rr % p.hpk;
        const float* qp = p.q + (size_t)(s * p.T + t) * p.q_tok + h * HD + 8 * g;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            qraw[rt][ds][0] = *reinterpret_cast<const float4v*>(qp + 32 * ds);
            qraw[rt][ds][1] = *reinterpret_cast<const float4v*>(qp + 32 * ds + 4);
        }
    }
    // (issued even with no block: past num_records they read zeros without
    // touching memory, and the compiler's wait for the queries is then the
    // same count on every path; such a wave waits for them before its K/V
    // buffer holds its state)
    if (QFIRST) {
        issue_k(0, true);
        issue_v(0, true);
        if (nb == 1) DTRACE(3);  // (one-block waves: stamp 3 = block 0 requested)
    }

    // ---- f16 parts (hi[, lo]) of the queries in base 2 ----
    // PK: column c16 < 8 holds the hi part of row c16, column c16 + 8 its lo
    // part; the two partial scores are summed across lanes l, l ^ 8.
    half8 qf[NP][RT][DS];
    int posr[RT], lor[RT];
    int lo_hi = 0, pos_lo = INT32_MAX;  // keys every valid row of the wave sees
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = rbase + 16 * rt + (PK ? (c16 & 7) : c16);
        const bool rv_ok = r < p.R;
        const int rr = rv_ok ? r : 0;
        const int t = rr / p.hpk;
        const KeyRange krg = key_range(p, len, t);
        posr[rt] = rv_ok ? krg.pos : -1;
        lor[rt] = krg.lo;
        if (rv_ok) {
            lo_hi = max(lo_hi, krg.lo);
            pos_lo = min(pos_lo, krg.pos);
        }
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const float4v a = qraw[rt][ds][0], b = qraw[rt][ds][1];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = rv_ok ? (j < 4 ? a[j] : b[j - 4]) * p.qscale : 0.f;
                const _Float16 hi = (_Float16)x;
                const _Float16 lo = (_Float16)(x - (float)hi);
                if (PK) {
                    qf[0][rt][ds][j] = c16 < 8 ? hi : lo;
                } else {
                    qf[0][rt][ds][j] = hi;
                    if (NP > 1) qf[NP - 1][rt][ds][j] = lo;
                }
            }
        }
    }
    if (W > 1) {
        // the arrival counters are set before any wave can count itself in
        if (tid < H) arrivals[tid] = 0;
        lds_barrier();
    }
    // wave-uniform bounds: blocks inside [lo_hi, pos_lo] need no mask
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        lo_hi = max(lo_hi, __shfl_xor(lo_hi, off, 64));
        pos_lo = min(pos_lo, __shfl_xor(pos_lo, off, 64));
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

    // A operand of k-step ds for key tile kt: key 16 kt + c16 (k_swz of it
    // is k_swz(c16)), logical piece g + 4 ds
    const char* kread[DS];
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) kread[ds] = klds + c16 * (HD * 2) + 16 * ((g + 4 * ds) ^ k_swz<HD>(c16));
    float4v sc[4][RT];
    // after_reads: runs once the block's K operands are in registers (the
    // K buffer is then free for the next block's loads)
    // The block's first 32 keys come with the first half of its loads: their
    // QK^T runs once that half has landed (the wait before qk), the second
    // half's after mid_wait() — the products overlap the block's arrival.
    auto qk = [&](auto&& mid_wait, auto&& after_reads) {
        half8 kc[4][DS];
        // independent accumulators per (part, key tile, row tile); the
        // k-steps run outermost so consecutive MFMAs do not depend on each other
        float4v acc[NP][4][RT];
#pragma unroll
        for (int pp = 0; pp < NP; ++pp)
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) acc[pp][kt][rt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            if (half == 1) mid_wait();
#pragma unroll
            for (int kt = 2 * half; kt < 2 * half + 2; ++kt)
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) kc[kt][ds] = load16(kread[ds] + kt * 16 * (HD * 2));
            if (half == 1) after_reads();
#pragma unroll
            for (int ds = 0; ds < DS; ++ds)
#pragma unroll
                for (int pp = 0; pp < NP; ++pp)
#pragma unroll
                    for (int kt = 2 * half; kt < 2 * half + 2; ++kt)
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt)
                            acc[pp][kt][rt] = mfma16(kc[kt][ds], qf[pp][rt][ds], acc[pp][kt][rt]);
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                if (PK) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) sc[kt][rt][i] = acc[0][kt][rt][i] + ror8(acc[0][kt][rt][i]);
                } else {
                    sc[kt][rt] = NP > 1 ? acc[0][kt][rt] + acc[NP - 1][kt][rt] : acc[0][kt][rt];
                }
            }
    };
    // The softmax needs only the scores: it runs before wait_v() (the wait
    // for the block's V), while V is still arriving.  EARLY_V (head dim 64:
    // 32 more VGPRs fit): the block's V^T operands are then all read and
    // after_vreads() runs before the PV MFMAs (the V buffer is free for the
    // next block's loads before PV, not after it).
    // wait_v_half(): keys 0-31 of the block's V landed (the first half of
    // its loads); wait_v(): all of it
    auto softmax_pv = [&](int kb, auto&& wait_v_half, auto&& wait_v, auto&& after_vreads) {
        const _Float16* vb = reinterpret_cast<const _Float16*>(vlds);
        // mask (blocks at a range boundary only): row r sees keys [lor, posr]
        if (kb < lo_hi || kb + 63 > pos_lo) {
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
        half8 pf[NPP][RT][2];
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
                    const _Float16 hi = (_Float16)pe;
                    const int e = (kt & 1) * 4 + i;
                    if (PK) {
                        pf[0][rt][kt >> 1][e] = c16 < 8 ? hi : (_Float16)(pe - (float)hi);
                    } else {
                        pf[0][rt][kt >> 1][e] = hi;
                        if (NPP > 1) pf[NPP - 1][rt][kt >> 1][e] = (_Float16)(pe - (float)hi);
                    }
                }
            l[rt] = l[rt] * c + ls;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt][rt] *= c;
        }
        // the softmax stays ahead of the wait for V (it needs only the
        // scores): the empty asm takes P as an operand, so P is computed
        // here; otherwise the compiler sinks the exp2s below the wait
#pragma unroll
        for (int pp = 0; pp < NPP; ++pp)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int u = 0; u < 2; ++u) __asm__ volatile("" : "+v"(pf[pp][rt][u]));
        // O^T += V^T P^T over keys 32 u .. 32 u + 31; the dim tiles are
        // independent accumulators.  Keys 0-31 go as soon as the first half
        // of V has landed.  EARLY_V: each half's V^T operands are all read
        // before its MFMAs, and the next block's V goes out after the
        // second half's reads.
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 0) wait_v_half();
            else wait_v();
            half8 va[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int k0 = 32 * u + 4 * g + (c16 >> 2), d0 = 16 * dt + 4 * (c16 & 3);
                va[dt] = cat8(lds_read_tr(v_elem<HD>(vb, k0, d0)), lds_read_tr(v_elem<HD>(vb, k0 + 16, d0)));
            }
            if (EARLY_V && u == 1) after_vreads();
#pragma unroll
            for (int pp = 0; pp < NPP; ++pp)
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) o[dt][rt] = mfma16(va[dt], pf[pp][rt][u], o[dt][rt]);
        }
    };

    // One block in flight per wave: K(i), V(i) are outstanding at the top
    // of trip i (in that order).  A buffer is refilled as soon as its reads
    // are done (lgkmcnt): K(i+1) after QK^T, V(i+1) after PV.  (Loads past
    // the wave's last block are not issued, so nothing is pending when the
    // state reuses the buffers.)
    // The vmcnt waits below are counted by hand from that order (VPL loads
    // per K or V block): the loop body, qk() and softmax_pv() must issue no
    // other vector-memory operation (no global or buffer load or store), or
    // a wait would return before its block has landed.  The loop's loads
    // are untracked by the compiler, which would otherwise wait for every
    // outstanding load (K(i+1) too) before PV's transposing V reads.
    for (int i = 0; i < nb; ++i) {
        wait_vm<VPL + VPL / 2>();  // the first half of K(i) landed
        if (i == 0) DTRACE(1);
        qk([&] { wait_vm<VPL>(); },  // K(i) landed
           [&] {
               wait_lgkm0();
               if (i + 1 < nb) issue_k(i + 1, false);
           });
        softmax_pv(
            blk(i),
            [&] {  // the first half of V(i) landed (K(i+1) may be in flight behind it)
                if (i + 1 < nb) wait_vm<VPL + VPL / 2>();
                else wait_vm<VPL / 2>();
            },
            [&] {
                if (i + 1 < nb) wait_vm<VPL>();  // V(i) landed
                else wait_vm<0>();
                if (i < 2) DTRACE(2 + i);
            },
            [&] {
                wait_lgkm0();
                if (i + 1 < nb) issue_v(i + 1, false);
            });
        if constexpr (!EARLY_V) {
            wait_lgkm0();
            if (i + 1 < nb) issue_v(i + 1, false);
        }
    }
    if (QFIRST && nb == 0) wait_vm<0>();  // (block 0's zero reads: the buffers hold the state next)
    DTRACE(4);
    if (PK) {
        // columns c16 and c16 ^ 8 hold the hi and lo parts of one row
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[dt][0][i] += ror8(o[dt][0][i]);
    }

    // ---- merge the W wave states of each head ----
    // No workgroup barrier: each wave leaves its state (m, l, O) in its own
    // K/V buffer (free after its last block) and counts itself in on its
    // head's LDS counter; the wave that arrives last merges the W states in
    // wave order and writes the result.  LDS operations of one wave complete
    // in order, so a wave's state is in place before its count.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) l[rt] = group4_sum(l[rt]);
    float4v* st_o = reinterpret_cast<float4v*>(klds);               // [DT][RT][64 lanes]
    float2* st_ml = reinterpret_cast<float2*>(klds + DT * RT * 64 * 16);  // [RT][64 lanes]
    auto state_of = [&](int w) {
        return reinterpret_cast<char*>(smem) + (w * H + hl) * WSLOT;
    };
    if (W > 1) {
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) st_o[(dt * RT + rt) * 64 + lane] = o[dt][rt];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) st_ml[rt * 64 + lane] = make_float2(m[rt], l[rt]);
        unsigned prev = 0;
        if (lane == 0)
            prev = __hip_atomic_fetch_add(&arrivals[hl], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
        prev = __builtin_amdgcn_readfirstlane(prev);
        if (prev != W - 1) {
            DTRACE(5);
            return;
        }
        // last of the head's waves: merge all W states in wave order
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float mw[W], lw[W];
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float2 ml = reinterpret_cast<const float2*>(state_of(w) + DT * RT * 64 * 16)[rt * 64 + lane];
                mw[w] = ml.x;
                lw[w] = ml.y;
                M = fmaxf(M, ml.x);
            }
            const float ms = (M == -INFINITY) ? 0.f : M;
            float L = 0.f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt][rt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float wt = fast_exp2(mw[w] - ms);
                L += lw[w] * wt;
                const float4v* so = reinterpret_cast<const float4v*>(state_of(w));
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[dt][rt] += so[(dt * RT + rt) * 64 + lane] * wt;
            }
            m[rt] = M;
            l[rt] = L;
        }
    }

    if (W > 1) DTRACE(5);  // (the merging wave: merge done)
    // this lane's result: row 16 rt + c16 (PK: c16 < 8), dims 16 dt + 4 g
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int row = 16 * rt + c16;
        const int r = rbase + row;
        if ((PK && c16 >= 8) || r >= p.R) continue;
        const float M = m[rt], L = l[rt];
        const int t = r / p.hpk, h = kvh * p.hpk + r % p.hpk;
        if (single && p.parts) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                store_part(p.parts + ((size_t)(s * p.T + t) * p.n_head + h) * (HD + 2), 16 * dt + 4 * g, M, L, o[dt][rt]);
        } else if (single) {
            // the only split: normalise here, sink in max and denominator
            const float ms = (M == -INFINITY) ? 0.f : M;
            float f;
            if (p.sinks) {
                const float sk = p.sinks[h] * kLog2e;
                const float M2 = fmaxf(M, sk);
                const float wgt = fast_exp2(ms - M2);
                f = wgt / (L * wgt + fast_exp2(sk - M2));
            } else {
                f = 1.f / L;
            }
            float* op = p.out + (size_t)(s * p.T + t) * p.o_tok + h * HD + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<float4v*>(op + 16 * dt) = o[dt][rt] * f;
        } else {
            const size_t idx = ((size_t)(s * p.n_kv + kvh) * p.R + r) * p.n_slot + slot;
            if constexpr (PART_WT) {
                // write-through (sc1): the partials reach the coherence point
                // as they are stored, not in the end-of-kernel write-back
                const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(p.ws_ml, (short)0, 0x7fffffff, kBufferFlags);
                const __amdgpu_buffer_rsrc_t rpo = __builtin_amdgcn_make_buffer_rsrc(p.ws_o, (short)0, 0x7fffffff, kBufferFlags);
                if (g == 0)
                    __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(M), __float_as_uint(L)}, rml, (int)(8 * idx), 0,
                                                          kPartWriteThrough);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[dt][rt]), rpo,
                                                           (int)(4 * (idx * HD + 16 * dt + 4 * g)), 0, kPartWriteThrough);
            } else {
                if (g == 0) *reinterpret_cast<float2*>(p.ws_ml + 2 * idx) = make_float2(M, L);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<float4v*>(p.ws_o + idx * HD + 16 * dt + 4 * g) = o[dt][rt];
            }
        }
    }
    DTRACE(6);
    };  // split

    if (!SK) {
        const int slot = blockIdx.x, by = blockIdx.y, s = blockIdx.z;
        const int len = seq_keys(p.seq_len, s, p.kv_len);
        if (len < p.T || len <= 0) return;
        const int kmax = min(len, p.kr_hi);  // keys past the last one of the call
        const int split0 = key_range(p, len, 0).lo / p.split_keys;
        const int n_active = min(p.n_slot, (kmax - 1) / p.split_keys - split0 + 1);
        if (slot >= n_active) return;
        const int kbeg = (split0 + slot) * p.split_keys;
        const int64_t row0 = p.seq_off ? p.seq_off[s] : (int64_t)s * (p.ring_cap ? p.ring_cap : p.kv_len);
        split(s, by, len, row0, kbeg, min(kbeg + p.split_keys, kmax), slot, n_active == 1);
        return;
    }
    // stream-K: this workgroup's range of the block list, piece by piece
    const int gy = hgroups * p.n_rg;
    const SeqTables tb = seq_tables(p);
    const SkLayout L = sk_layout(p, gy, tb);
    const int w = blockIdx.x;
    if (w >= L.g_eff || L.total == 0) return;
    int cur = L.start(w);
    const int end = L.start(w + 1);
    if (cur >= end) return;
    // the sequence holding position cur (< total, so some lane of the scan
    // finds it), and the positions before it
    int s = 0;
    int pre = 0;  // positions before sequence s
    for (int base = 0; base < p.n_seq; base += 64) {
        const int x = base + lane < p.n_seq ? sk_span_of(p, tb.keys_lane(p, base + lane)) * gy : 0;
        int incl = x;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(incl, off, 64);
            if (lane >= off) incl += y;
        }
        const unsigned long long hit = __builtin_amdgcn_ballot_w64(pre + incl > cur);
        if (hit) {
            const int j = __builtin_ctzll(hit);
            s = base + j;
            pre = uniform32(pre + __shfl(incl - x, j, 64));
            break;
        }
        pre = uniform32(pre + __shfl(incl, 63, 64));
    }
    while (cur < end && s < p.n_seq) {
        const int len = uniform32(tb.keys(p, s));
        const int nb = sk_blocks_of(p, len);
        const int span = nb ? nb + p.sk_restart : 0;
        if (nb == 0 || cur >= pre + span * gy) {  // past this sequence
            pre += span * gy;
            ++s;
            continue;
        }
        const int by = (cur - pre) / span;
        const int seg = pre + by * span + p.sk_restart;  // the segment's first block
        if (cur < seg) {  // (in the start-up positions)
            cur = seg;
            if (cur >= end) break;
        }
        const int pend = min(end, seg + nb);
        const int slot = w - L.owner(seg);
        // the segment's first piece records how many pieces it has
        if (slot == 0 && p.ws_np && tid == 0) p.ws_np[s * gy + by] = L.owner(seg + nb - 1) - w + 1;
        split(s, by, len, tb.row0(p, s), 64 * (cur - seg), min(64 * (pend - seg), len), slot,
              cur == seg && pend == seg + nb);
        // the next piece reuses the LDS buffers and counters
        __syncthreads();
        cur = pend;
    }
}

// Combine of the split partials of one query row, in key order, with the
// head's sink (merge_dec, src/moe_kernels.rs:585-617; ATTN_M,
// src/oss_batch.rs:395-425).  Grid (R x dim quarters, n_kv, n_seq), 256
// threads; thread (phase, 4-dim chunk) merges the splits c = phase (mod
// phases) online (running max, rescaled sum), all of its loads in flight
// at once; the phases of a wave merge through lane exchanges, the four
// waves through LDS, in a fixed order; head dim 128 takes four workgroups
// per row (32 dims each).  ROW_WAVES: one wave per row (four rows per
// workgroup, grid x = R / 4), for rows with few splits (<= 16): no LDS
// stage, a quarter of the workgroups.
// dims per combine workgroup (DW): hd 128 in four slices of 32 (calls of
// C2's size have only rows x kv heads = 32 rows: four times the workgroups
// load the partials, 11.5 -> 11.3 us); hd 512 (MLA) in slices of 32 for
// calls of <= 32 rows (16 heads x 32K latent rows: 18.9 -> 17.1 us), else
// of 128 (a 64-token chunk has only 4 splits a row: slices of 32 leave most
// threads idle, 102 -> 138 us)
template <int HD, bool ROW_WAVES, int DW>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams p) {
    static_assert(!ROW_WAVES || HD <= 128, "one wave covers the row's dims");
    static_assert((HD % DW == 0 && DW % 32 == 0) || DW == HD, "dims split into whole slices");
    constexpr int NQ = HD / DW;
    constexpr int D4 = DW / 4;
    // phases: 256 / (DW / 4) (16 at hd 64, 32 at DW 32); one wave per row: 4, 2
    constexpr int PH = (ROW_WAVES ? 64 : 256) / D4;
    constexpr int J = DW < 128 && HD >= 128 ? 4 : 8;  // splits per thread per pass
    __shared__ float4v s_o[4][D4];
    __shared__ float2 s_ml[4][D4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pt = ROW_WAVES ? lane : tid;  // this thread's index within its row
    const int r = ROW_WAVES ? blockIdx.x * 4 + wave : blockIdx.x / NQ, dq = ROW_WAVES ? 0 : blockIdx.x % NQ;
    const int kvh = blockIdx.y, s = blockIdx.z;
    if (ROW_WAVES && r >= p.R) return;
    const int len = seq_keys(p.seq_len, s, p.kv_len);
    if (len < p.T || len <= 0) return;
    const int t = r / p.hpk, h = kvh * p.hpk + r % p.hpk;
    int c0, c1;  // the splits that hold keys of this row
    if (p.sk_grid > 0) {
        // stream-K: every piece of the row's segment (rows with no key in a
        // piece have an empty partial there); the split kernel records the
        // count.  (Loading every workspace slot before the count arrives was
        // measured slower: 12.6 vs 11.7 us on a 32-sequence draft batch.)
        const int hgroups = p.n_kv / p.wg_heads;
        c0 = 0;
        c1 = p.ws_np[s * hgroups * p.n_rg + (r / p.rg_rows) * hgroups + kvh / p.wg_heads] - 1;
        if (c1 < 1) return;  // one piece: the split kernel wrote the output
    } else {
        const int split0 = key_range(p, len, 0).lo / p.split_keys;
        const int n_active = min(p.n_slot, (min(len, p.kr_hi) - 1) / p.split_keys - split0 + 1);
        if (n_active <= 1) return;  // the split kernel wrote the output
        const KeyRange krg = key_range(p, len, t);
        c0 = krg.lo / p.split_keys - split0;
        c1 = min(krg.pos / p.split_keys - split0, n_active - 1);
    }
    const size_t base = ((size_t)(s * p.n_kv + kvh) * p.R + r) * p.n_slot;
    const int ph = pt / D4, d = 4 * (pt % D4) + DW * dq;
    // the sink logit is requested now, not after the merge
    const float sk = (p.sinks && !p.parts && pt < D4) ? p.sinks[h] * kLog2e : -INFINITY;

    float m = -INFINITY, l = 0.f;
    float4v o = {0.f, 0.f, 0.f, 0.f};
    for (int cb = c0; cb <= c1; cb += PH * J) {
        float2 ml[J];
        float4v ov[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = cb + ph + PH * j;
            const bool ld = c <= c1;
            ml[j] = ld ? *reinterpret_cast<const float2*>(p.ws_ml + 2 * (base + c)) : make_float2(-INFINITY, 0.f);
            ov[j] = ld ? *reinterpret_cast<const float4v*>(p.ws_o + (base + c) * HD + d) : float4v{0.f, 0.f, 0.f, 0.f};
        }
        float mb = m;
#pragma unroll
        for (int j = 0; j < J; ++j) mb = fmaxf(mb, ml[j].x);
        const float ms = (mb == -INFINITY) ? 0.f : mb;
        const float f = fast_exp2(m - ms);
        l *= f;
        o *= f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float w = fast_exp2(ml[j].x - ms);
            l += ml[j].y * w;
            o += ov[j] * w;
        }
        m = mb;
    }
    // merge (m, l, o) states: a then b
    auto merge = [](float& m, float& l, float4v& o, float m2, float l2, const float4v& o2) {
        const float M = fmaxf(m, m2);
        const float ms = (M == -INFINITY) ? 0.f : M;
        const float a = fast_exp2(m - ms), b = fast_exp2(m2 - ms);
        l = l * a + l2 * b;
        o = o * a + o2 * b;
        m = M;
    };
    // Exchange with lane ^ off (off = 16 or 32) by permlane swaps (no LDS):
    // each lane gets the pair (value of the lower lane, value of the upper).
    auto pair = [](float x, int off) {
        if (off < 16) {  // (the lane off apart, through the LDS crossbar)
            const float y = __shfl_xor(x, off, 64);
            const bool upper = (threadIdx.x & off) != 0;
            return upper ? make_float2(y, x) : make_float2(x, y);
        }
        const auto v = off == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                                 : __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
    };
#pragma unroll
    for (int off = D4; off < 64; off <<= 1) {
        // lower phase first; both lanes compute the same merge
        const float2 mp = pair(m, off), lp = pair(l, off);
        float4v olo, ohi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 op = pair(o[i], off);
            olo[i] = op.x;
            ohi[i] = op.y;
        }
        m = mp.x;
        l = lp.x;
        o = olo;
        merge(m, l, o, mp.y, lp.y, ohi);
    }
    if (!ROW_WAVES) {
        if (lane < D4) {
            s_o[wave][lane] = o;
            s_ml[wave][lane] = make_float2(m, l);
        }
        __syncthreads();
    }
    if (pt < D4) {
        float M = m, L = l;
        float4v O = o;
        if (!ROW_WAVES) {
            M = s_ml[0][tid].x;
            L = s_ml[0][tid].y;
            O = s_o[0][tid];
#pragma unroll
            for (int w = 1; w < 4; ++w) merge(M, L, O, s_ml[w][tid].x, s_ml[w][tid].y, s_o[w][tid]);
        }
        if (p.parts) {
            store_part(p.parts + ((size_t)(s * p.T + t) * p.n_head + h) * (HD + 2), d, M, L, O);
        } else {
            // sink: in the max and the denominator
            float f = 1.f / L;
            if (p.sinks) {
                const float M2 = fmaxf(M, sk);
                const float ms = (M == -INFINITY) ? 0.f : M;
                const float wgt = fast_exp2(ms - M2);
                f = wgt / (L * wgt + fast_exp2(sk - M2));
            }
            *reinterpret_cast<float4v*>(p.out + (size_t)(s * p.T + t) * p.o_tok + h * HD + d) = O * f;
        }
    }
}

template <int HD, int RT, int NW, int H>
static hipError_t launch_k(const DecodeParams& p, hipStream_t st) {
    dim3 grid(p.n_slot, p.n_kv / p.wg_heads * p.n_rg, p.n_seq);
    {
    ProfScope ps(kProfDecodeSplit, st);
    // up to 8 rows per kv head: hi and lo parts share one MFMA (packed columns)
    const bool pk = RT == 1 && p.R <= 8;
    if (p.sk) {
        // (the planner's stream-K shapes: 4 waves on one kv head, up to 32
        // rows per kv head at head dim 64)
        if constexpr (H == 1 && NW == 4 && !(HD == 64 && RT == 4)) {
            if (p.ring_cap || p.window || !p.seq_len) return hipErrorInvalidValue;
            if (pk) hipLaunchKernelGGL((decode_kernel<HD, RT, NW, H, false, RT == 1, true>), dim3(p.sk_grid), dim3(64 * NW), 0, st, p);
            else hipLaunchKernelGGL((decode_kernel<HD, RT, NW, H, false, false, true>), dim3(p.sk_grid), dim3(64 * NW), 0, st, p);
        } else {
            return hipErrorInvalidValue;
        }
    } else if (p.ring_cap) {
        if (pk) hipLaunchKernelGGL((decode_kernel<HD, RT, NW, H, true, RT == 1, false>), grid, dim3(64 * NW), 0, st, p);
        else hipLaunchKernelGGL((decode_kernel<HD, RT, NW, H, true, false, false>), grid, dim3(64 * NW), 0, st, p);
    } else {
        if (pk) hipLaunchKernelGGL((decode_kernel<HD, RT, NW, H, false, RT == 1, false>), grid, dim3(64 * NW), 0, st, p);
        else hipLaunchKernelGGL((decode_kernel<HD, RT, NW, H, false, false, false>), grid, dim3(64 * NW), 0, st, p);
    }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.n_slot == 1 || p.split_only) return e;
    return launch_combine(p, st);
}

// rows with at most this many splits take the one-wave-per-row combine
constexpr int kCombineRowWaveSlots = 16;

hipError_t launch_combine(const DecodeParams& p, hipStream_t st) {
    ProfScope ps(kProfDecodeCombine, st);
    if (p.hd <= 128 && p.n_slot <= kCombineRowWaveSlots) {
        const dim3 grid((p.R + 3) / 4, p.n_kv, p.n_seq);
        if (p.hd == 64) hipLaunchKernelGGL((decode_combine_kernel<64, true, 64>), grid, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((decode_combine_kernel<128, true, 128>), grid, dim3(256), 0, st, p);
        return hipGetLastError();
    }
    auto grid = [&](int dw) { return dim3(p.R * (p.hd / dw), p.n_kv, p.n_seq); };
    switch (p.hd) {
        case 64: hipLaunchKernelGGL((decode_combine_kernel<64, false, 64>), grid(64), dim3(256), 0, st, p); break;
        case 128: hipLaunchKernelGGL((decode_combine_kernel<128, false, 32>), grid(32), dim3(256), 0, st, p); break;
        case 512:
            if ((long long)p.R * p.n_seq <= 32)
                hipLaunchKernelGGL((decode_combine_kernel<512, false, 32>), grid(32), dim3(256), 0, st, p);
            else
                hipLaunchKernelGGL((decode_combine_kernel<512, false, 128>), grid(128), dim3(256), 0, st, p);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_decode(const DecodeParams& p, int rt, int nw, hipStream_t st) {
    if (p.hd == 64) {
        if (nw == 8 && p.wg_heads == 4) {
            if (rt == 1) return launch_k<64, 1, 8, 4>(p, st);
            if (rt == 2) return launch_k<64, 2, 8, 4>(p, st);
        } else if (nw == 4 && p.wg_heads == 1) {
            if (rt == 1) return launch_k<64, 1, 4, 1>(p, st);
            if (rt == 2) return launch_k<64, 2, 4, 1>(p, st);
            if (rt == 4) return launch_k<64, 4, 4, 1>(p, st);
        }
    } else if (p.hd == 128 && nw == 4 && p.wg_heads == 1) {
        if (rt == 1) return launch_k<128, 1, 4, 1>(p, st);
        if (rt == 2) return launch_k<128, 2, 4, 1>(p, st);
    } else if (p.hd == 128 && nw == 1 && p.wg_heads == 1) {
        if (rt == 1) return launch_k<128, 1, 1, 1>(p, st);
        if (rt == 2) return launch_k<128, 2, 1, 1>(p, st);
    }
    return hipErrorInvalidValue;
}

// fill kernel for the workspace counters (graph-capturable, no memset node)
__global__ void zero_u32_kernel(unsigned* p, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

#ifdef PELICA_DTRACE
extern "C" int pelica_attn_debug_trace(void* dst, size_t bytes) {
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_dtrace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

hipError_t launch_zero(unsigned* p, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(zero_u32_kernel, dim3(blocks), dim3(256), 0, st, p, n);
    return hipGetLastError();
}

}  // namespace pelica
