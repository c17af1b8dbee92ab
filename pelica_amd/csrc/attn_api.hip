// The C ABI of libpelica_attn.so (include/pelica_attn.h): descriptor
// validation, split planning, launches, and the partials merge kernel.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>

#include "../../include/pelica_attn.h"
#include "attn_decode.hpp"
#include "attn_merge.hpp"
#include "attn_prefill.hpp"
#include "attn_qkv.hpp"
#include "attn_prof.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    if (!s || !*s) return dflt;
    return atoi(s);
}

// The planner's tuning switches, read from the environment once per process
// (at the first call that plans a decode or MLA pass): the plan, and with it
// the workspace size, cannot change between calls.  0 = unset.
struct Tuning {
    bool streamk;       // PELICA_ATTN_STREAMK (default 1)
    int split_blocks;   // PELICA_ATTN_SPLIT_BLOCKS (64-key blocks per wave; > 0 also turns stream-K off)
    int decode_waves;   // PELICA_ATTN_DECODE_WAVES (target waves of a split grid)
    int sk_restart;     // PELICA_ATTN_SK_RESTART (positions charged per stream-K piece start)
    int mla_workgroups; // PELICA_ATTN_MLA_WORKGROUPS
};

Tuning read_tuning() {
    Tuning x;
    x.streamk = env_int("PELICA_ATTN_STREAMK", 1) != 0;
    x.split_blocks = std::max(0, env_int("PELICA_ATTN_SPLIT_BLOCKS", 0));
    x.decode_waves = std::max(0, env_int("PELICA_ATTN_DECODE_WAVES", 0));
    x.sk_restart = env_int("PELICA_ATTN_SK_RESTART", -1);
    x.mla_workgroups = std::max(0, env_int("PELICA_ATTN_MLA_WORKGROUPS", 0));
    return x;
}

// Published as an immutable object through an atomic pointer, so a reload
// never races a planning call; a replaced object is kept (a planning call
// may still read it), a few bytes per reload.
std::atomic<const Tuning*> g_tuning{nullptr};

const Tuning& tuning() {
    const Tuning* t = g_tuning.load(std::memory_order_acquire);
    if (!t) {
        const Tuning* fresh = new Tuning(read_tuning());
        if (g_tuning.compare_exchange_strong(t, fresh, std::memory_order_acq_rel)) t = fresh;
        else delete fresh;  // another thread published first: t is its object
    }
    return *t;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

// compute units of the current device (queried once per process)
long long device_cus() {
    static const long long n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;  // MI355X
        return (long long)cus;
    }();
    return n;
}

int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

// Checks shared by decode and prefill.
// mla: the latent layout (hd 512, one kv head, no window or ring)
int check_desc(const PelicaAttnDesc* d, bool mla = false) {
    if (!d) return fail(PELICA_ATTN_EINVAL, "desc is NULL");
    if (d->flags & ~PELICA_ATTN_FLAG_SPLIT_ONLY) return fail(PELICA_ATTN_EINVAL, "unknown flags %u", d->flags);
    if (d->n_head <= 0 || d->n_kv <= 0 || d->n_head % d->n_kv)
        return fail(PELICA_ATTN_EINVAL, "n_head %d must be a positive multiple of n_kv %d", d->n_head, d->n_kv);
    if (mla) {
        if (d->hd != 512 || d->n_kv != 1 || d->window || d->ring_cap)
            return fail(PELICA_ATTN_EUNSUPPORTED, "MLA takes hd 512, n_kv 1, no window or ring");
    } else if (d->hd != 64 && d->hd != 128) {
        return fail(PELICA_ATTN_EUNSUPPORTED, "hd %d unsupported (64 or 128)", d->hd);
    }
    if (d->n_seq <= 0 || d->q_tokens <= 0)
        return fail(PELICA_ATTN_EINVAL, "n_seq %d and q_tokens %d must be positive", d->n_seq, d->q_tokens);
    if (d->kv_len < d->q_tokens)
        return fail(PELICA_ATTN_EINVAL, "kv_len %d is below q_tokens %d (the queries' own keys are in the cache)",
                    d->kv_len, d->q_tokens);
    if (d->window < 0 || d->ring_cap < 0)
        return fail(PELICA_ATTN_EINVAL, "window %d and ring_cap %d must be >= 0", d->window, d->ring_cap);
    if (d->kv_row_stride != 0 && d->kv_row_stride < (int64_t)d->n_kv * d->hd)
        return fail(PELICA_ATTN_EINVAL, "kv_row_stride %lld is below n_kv*hd", (long long)d->kv_row_stride);
    if (d->kv_row_stride % 8)
        return fail(PELICA_ATTN_EINVAL, "kv_row_stride must be a multiple of 8 values (16-byte rows)");
    if (d->ring_cap) {
        // every key a token of the pass sees must still be in the ring
        const int pos0 = d->kv_len - d->q_tokens;
        const int lo0 = (d->window > 0 && pos0 + 1 > d->window) ? pos0 + 1 - d->window : 0;
        if (d->kv_len - lo0 > d->ring_cap)
            return fail(PELICA_ATTN_EINVAL, "ring_cap %d cannot hold the %d keys the pass sees", d->ring_cap,
                        d->kv_len - lo0);
    }
    if (!(d->scale >= 0.f) || std::isinf(d->scale)) return fail(PELICA_ATTN_EINVAL, "scale must be finite, >= 0");
    {
        // one sequence's rows of one kv head are addressed with 32-bit byte offsets
        const long long stride = d->kv_row_stride ? d->kv_row_stride : (long long)d->n_kv * d->hd;
        const long long rows = (d->ring_cap ? d->ring_cap : d->kv_len) + 128LL;
        if (rows * stride * 2 >= (1LL << 32))
            return fail(PELICA_ATTN_EUNSUPPORTED, "a sequence's cache span (%lld rows x %lld values) exceeds 4 GiB",
                        rows - 128, stride);
    }
    return PELICA_ATTN_OK;
}

// Token strides of q and out (values of q_es / o_es bytes): 0 or at least a
// token's heads, keeping every token's rows 16-byte aligned, and below 2^20
// values (the kernels address a block of tokens with 32-bit byte offsets).
int check_strides(const PelicaAttnDesc* d, int q_es, int o_es) {
    const int64_t row = (int64_t)d->n_head * d->hd;
    auto bad = [&](int64_t st, int es) { return st != 0 && (st < row || st >= (1 << 20) || (st * es) % 16); };
    if (bad(d->q_token_stride, q_es))
        return fail(PELICA_ATTN_EINVAL, "q_token_stride %lld: 0, or >= n_head*hd (%lld), < 2^20 and a whole number of "
                    "16-byte pieces", (long long)d->q_token_stride, (long long)row);
    if (bad(d->out_token_stride, o_es))
        return fail(PELICA_ATTN_EINVAL, "out_token_stride %lld: 0, or >= n_head*hd (%lld), < 2^20 and a whole number "
                    "of 16-byte pieces", (long long)d->out_token_stride, (long long)row);
    return PELICA_ATTN_OK;
}

int64_t q_stride(const PelicaAttnDesc* d) { return d->q_token_stride ? d->q_token_stride : (int64_t)d->n_head * d->hd; }
int64_t o_stride(const PelicaAttnDesc* d) { return d->out_token_stride ? d->out_token_stride : (int64_t)d->n_head * d->hd; }

float eff_scale(const PelicaAttnDesc* d) { return d->scale > 0.f ? d->scale : 1.f / std::sqrt((float)d->hd); }

struct DecodePlan {
    int R, rt, n_rg, split_keys, n_slot, wg_heads, nw;
    bool sk;
    int sk_grid, sk_minb, sk_restart;
    size_t ctr_bytes, ml_bytes, o_bytes, ws_bytes;
};

// kr_len: keys of the call's key range (pelica_attn_decode_partials_range),
// 0 for the whole cache
int plan_decode(const PelicaAttnDesc* d, DecodePlan* pl, int kr_len = 0) {
    int rc = check_desc(d);
    if (rc) return rc;
    const Tuning& tn = tuning();
    const int hpk = d->n_head / d->n_kv;
    const int R = d->q_tokens * hpk;
    int rt;
    if (d->hd == 64) rt = R <= 16 ? 1 : R <= 32 ? 2 : 4;
    else rt = R <= 16 ? 1 : 2;
    const int n_rg = ceil_div(R, 16 * rt);
    // keys any row of a sequence can see
    const long long span = d->window > 0 ? std::min<long long>(d->kv_len, (long long)d->window + d->q_tokens - 1)
                                         : d->kv_len;
    // A key range plans the splits of the whole cache (the same split size,
    // so its workspace is never larger than pelica_attn_workspace_bytes
    // gives) and keeps the splits that hold its keys.
    const long long span_r = kr_len > 0 ? std::min<long long>(span, kr_len) : span;
    const bool bounded = d->window > 0 || kr_len > 0;
    const long long groups = (long long)d->n_seq * d->n_kv * n_rg;
    const long long blocks = (long long)ceil_div(span, 64) * groups;
    // Workgroup shape.  Large head-dim-64 calls: 8 waves, 4 kv heads per
    // workgroup (2 waves each), ~2 waves per SIMD — the heads' slices of a
    // cache row are then read together (measured ~1 us faster on the 32K
    // gpt-oss layer).  Otherwise 4 waves on one kv head, ~1 wave per SIMD.
    // Ragged batches without window or ring go stream-K: a fixed grid shares
    // the batch's blocks evenly, whatever the spread of the lengths (with
    // one split grid the longest sequences' workgroups set the time)
    // (the kernel counts list positions in 32 bits: at most 2^31 - 1, with
    // every sequence at kv_len and the start-up charge)
    const int sk_restart = tn.sk_restart >= 0 ? tn.sk_restart : 8;
    const long long sk_positions =
        groups * ((long long)ceil_div(d->kv_len, 64) + sk_restart);
    const bool sk = d->seq_kv_len && d->window == 0 && d->ring_cap == 0 && !(d->hd == 64 && rt == 4) &&
                    tn.streamk && tn.split_blocks == 0 && sk_positions < 0x7fffffffLL;
    const bool big = !sk && pelica::decode_can_use_8_waves(d->hd, rt) && blocks >= 2048 && d->n_kv % 4 == 0;
    const int wg_heads = big ? 4 : 1;
    // 64-key blocks per wave: enough waves for every SIMD, each streaming
    // several blocks, so the split count (and the combine's work) stays small
    const int target_waves = std::max(64, tn.decode_waves ? tn.decode_waves : (big ? 2048 : 1024));
    int spw = tn.split_blocks;
    if (spw <= 0) spw = (int)std::max<long long>(1, (blocks + target_waves - 1) / target_waves);
    auto splits = [&](int nw_, long long* keys, int* ns) {
        long long split_keys = 64LL * (nw_ / wg_heads) * spw;
        int n_slot = 0;
        for (;;) {
            const int total = ceil_div(d->kv_len, split_keys);
            n_slot = bounded ? std::min<int>(total, ceil_div(span_r, split_keys) + 1) : total;
            if (n_slot <= pelica::kMaxSlots) break;
            split_keys *= 2;
        }
        *keys = split_keys;
        *ns = n_slot;
    };
    int nw = big ? 8 : 4;
    long long split_keys;
    int n_slot;
    splits(nw, &split_keys, &n_slot);
    // Small head-dim-128 calls: with 4-wave workgroups the grid would not
    // reach every CU (a CU pulls ~22 GB/s at most here), so split the keys
    // four times as finely over one-wave workgroups: every wave writes its
    // own split's partials, with no merge between waves after its last
    // block (OLMoE 2K / Qwen3 8K decode: split kernel 7.45 -> 6.97 /
    // 7.68 -> 6.88 us against 2-wave workgroups, whole call 10.14 -> 9.95
    // / 10.87 -> 10.45 us).
    if (!big && d->hd == 128 && (long long)n_slot * groups < device_cus()) {
        nw = 1;
        splits(nw, &split_keys, &n_slot);
    }
    // Window layers: when the keys any row sees fit one workgroup (each wave
    // <= 2 blocks), one split per kv head — the workgroup merges its waves
    // and writes the output itself, no combine launch.
    if (d->window > 0 && !big && (ceil_div(span, 64) + 1) <= 2 * (nw / wg_heads) &&
        tn.split_blocks == 0) {
        split_keys = ((long long)d->kv_len + 63) / 64 * 64;
        n_slot = 1;
    }
    pl->sk = sk;
    pl->sk_grid = pl->sk_minb = pl->sk_restart = 0;
    if (sk) {
        // one 4-wave workgroup per CU (two where two waves per SIMD fit:
        // head dim 64, one row tile);
        // ranges of at least minb blocks, and a bound on the pieces of one
        // segment (a sequence's blocks of one kv head and row group) for
        // the workspace: its blocks / minb + 1
        nw = 4;
        const int per_cu = (d->hd == 64 && rt == 1) ? 2 : 1;
        pl->sk_grid = (int)(device_cus() * per_cu);
        // (a piece's start-up is charged as sk_restart blocks: ~15 us of
        // pipeline refill against ~1.4 us per block of a workgroup's
        // stream; 8 measured best, 6-14 within 1.5 %)
        const int restart = sk_restart;
        const int maxblk = ceil_div(d->kv_len, 64);
        const long long bmax = (long long)d->n_seq * d->n_kv * n_rg * (maxblk + restart);
        int minb = (int)std::min<long long>(64, std::max<long long>(4, bmax / (2LL * pl->sk_grid)));
        while (ceil_div(maxblk + restart, minb) + 1 > pelica::kMaxSlots) minb *= 2;
        pl->sk_minb = minb;
        pl->sk_restart = restart;
        split_keys = 64;
        n_slot = std::min(maxblk, ceil_div(maxblk + restart, minb) + 1);
    }
    pl->R = R;
    pl->rt = rt;
    pl->n_rg = n_rg;
    pl->split_keys = (int)split_keys;
    pl->n_slot = n_slot;
    pl->wg_heads = wg_heads;
    pl->nw = nw;
    // workspace: (max, sum) pairs, then O rows, 256-byte aligned parts
    const size_t n_part = (size_t)d->n_seq * d->n_kv * R * n_slot;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    // stream-K: the piece count of each segment, then the partials
    pl->ctr_bytes = sk ? al((size_t)d->n_seq * d->n_kv * n_rg * 4) : 0;
    pl->ml_bytes = al(n_part * 2 * 4);
    pl->o_bytes = al(n_part * d->hd * 4);
    pl->ws_bytes = n_slot > 1 ? pl->ctr_bytes + pl->ml_bytes + pl->o_bytes : 0;
    return PELICA_ATTN_OK;
}

// MLA: rows = tokens x heads in row groups of 16, 32-key latent blocks.
// Measured on MI355X (32K-128K latent rows, 16-4096 rows): two workgroups
// per CU (512) is fastest while that leaves each workgroup >= 8 blocks,
// else one per CU (256); a split shorter than 128 keys loses more to its
// partials (2 KB a row) than it gains.
int plan_mla(const PelicaAttnDesc* d, DecodePlan* pl) {
    int rc = check_desc(d, true);
    if (rc) return rc;
    const int R = d->q_tokens * d->n_head;
    const int rt = 1;
    const int n_rg = ceil_div(R, 16 * rt);
    const long long blocks = (long long)ceil_div(d->kv_len, 32) * n_rg * d->n_seq;
    long long split_keys;
    if (tuning().mla_workgroups) {
        split_keys = 32LL * std::max<long long>(1, ceil_div(blocks, tuning().mla_workgroups));
    } else {
        const long long target = blocks >= 8 * 512 ? 512 : 256;
        split_keys = std::max<long long>(128, 32LL * ceil_div(blocks, target));
    }
    int n_slot = ceil_div(d->kv_len, split_keys);
    while (n_slot > pelica::kMaxSlots) {
        split_keys *= 2;
        n_slot = ceil_div(d->kv_len, split_keys);
    }
    pl->R = R;
    pl->rt = rt;
    pl->n_rg = n_rg;
    pl->split_keys = (int)split_keys;
    pl->n_slot = n_slot;
    pl->wg_heads = 1;
    pl->nw = 4;
    pl->sk = false;
    const size_t n_part = (size_t)d->n_seq * R * n_slot;
    pl->ctr_bytes = 0;
    pl->ml_bytes = (n_part * 2 * 4 + 255) & ~(size_t)255;
    pl->ws_bytes = n_slot > 1 ? pl->ml_bytes + n_part * 512 * 4 : 0;
    return PELICA_ATTN_OK;
}

}  // namespace

extern "C" {

int pelica_attn_version(void) { return PELICA_ATTN_VERSION; }

int pelica_attn_reload_tuning(void) {
    g_err[0] = 0;
    g_tuning.store(new Tuning(read_tuning()), std::memory_order_release);
    return PELICA_ATTN_OK;
}

const char* pelica_attn_last_error(void) { return g_err; }

size_t pelica_attn_workspace_bytes(const PelicaAttnDesc* desc) {
    g_err[0] = 0;
    DecodePlan pl;
    if (plan_decode(desc, &pl)) return 0;
    return pl.ws_bytes;
}

int pelica_attn_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    if (!workspace || workspace_bytes == 0) return PELICA_ATTN_OK;
    if (misaligned(workspace)) return fail(PELICA_ATTN_EINVAL, "workspace must be 16-byte aligned");
    hipError_t e = pelica::launch_zero(static_cast<unsigned*>(workspace), workspace_bytes / 4,
                                       static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(PELICA_ATTN_EHIP, "workspace init: %s", hipGetErrorString(e));
    return PELICA_ATTN_OK;
}

}  // extern "C"

namespace {

// decode into out (final, with sinks) or into merge_dec partial slots
// key_end > 0: keys [key_begin, key_end) only, cache row 0 = position key_begin
int run_decode(const PelicaAttnDesc* desc, const float* q, const uint16_t* k, const uint16_t* v,
               const float* sinks, float* out, float* parts, void* workspace, size_t workspace_bytes,
               void* stream, int key_begin = 0, int key_end = 0) {
    g_err[0] = 0;
    DecodePlan pl;
    int rc = plan_decode(desc, &pl, key_end > 0 ? key_end - key_begin : 0);
    if (rc) return rc;
    rc = check_strides(desc, 4, 4);
    if (rc) return rc;
    if (!q || !k || !v || !(out || parts))
        return fail(PELICA_ATTN_EINVAL, "q, k, v and %s must be non-NULL", parts ? "parts" : "out");
    if (parts && desc->flags) return fail(PELICA_ATTN_EINVAL, "flags must be 0");
    if (misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out) || misaligned(workspace))
        return fail(PELICA_ATTN_EINVAL, "q, k, v, out and workspace must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(parts) % 8) return fail(PELICA_ATTN_EINVAL, "parts must be 8-byte aligned");
    if (pl.ws_bytes && (!workspace || workspace_bytes < pl.ws_bytes))
        return fail(PELICA_ATTN_EWORKSPACE, "workspace of %zu bytes needed, %zu given", pl.ws_bytes,
                    workspace ? workspace_bytes : (size_t)0);
    pelica::DecodeParams p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.sinks = sinks;
    p.out = out;
    char* ws = static_cast<char*>(workspace);
    p.ws_ml = pl.ws_bytes ? reinterpret_cast<float*>(ws + pl.ctr_bytes) : nullptr;
    p.ws_o = pl.ws_bytes ? reinterpret_cast<float*>(ws + pl.ctr_bytes + pl.ml_bytes) : nullptr;
    p.seq_len = desc->seq_kv_len;
    p.seq_off = desc->seq_kv_offset;
    p.row_stride = desc->kv_row_stride ? desc->kv_row_stride : (int64_t)desc->n_kv * desc->hd;
    p.q_tok = q_stride(desc);
    p.o_tok = o_stride(desc);
    p.kr_lo = key_end > 0 ? key_begin : 0;
    p.kr_hi = key_end > 0 ? key_end : INT32_MAX;
    p.kv_len = desc->kv_len;
    p.n_head = desc->n_head;
    p.n_kv = desc->n_kv;
    p.hd = desc->hd;
    p.hpk = desc->n_head / desc->n_kv;
    p.T = desc->q_tokens;
    p.R = pl.R;
    p.n_rg = pl.n_rg;
    p.n_seq = desc->n_seq;
    p.window = desc->window;
    p.ring_cap = desc->ring_cap;
    p.qscale = eff_scale(desc) * pelica::kLog2e;
    p.n_slot = pl.n_slot;
    p.split_keys = pl.split_keys;
    p.wg_heads = pl.wg_heads;
    p.parts = parts;
    p.split_only = (desc->flags & PELICA_ATTN_FLAG_SPLIT_ONLY) != 0;
    p.sk = pl.sk;
    p.sk_grid = pl.sk_grid;
    p.sk_minb = pl.sk_minb;
    p.sk_restart = pl.sk_restart;
    p.rg_rows = 16 * pl.rt;
    p.ws_np = pl.sk && pl.ws_bytes ? reinterpret_cast<int*>(ws) : nullptr;
    hipError_t e = pelica::launch_decode(p, pl.rt, pl.nw, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(PELICA_ATTN_EHIP, "decode launch: %s", hipGetErrorString(e));
    return PELICA_ATTN_OK;
}

// Scratch of pelica_attn_decode_noalloc: a file-scope device array, one
// copy per GPU the library runs on, held until the process ends.  In host
// code `scratch` names a host-side stand-in, never the device memory: host
// code uses only the per-device address from hipGetSymbolAddress below.
static __device__ __align__(256) char scratch[PELICA_ATTN_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// This device's copy of `scratch`, looked up on the first call on the device
// (with that device current) and kept.
int scratch_of_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(PELICA_ATTN_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(PELICA_ATTN_EUNSUPPORTED, "device %d (at most %d)", dev, kMaxDevices);
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_acquire);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p)
                return fail(PELICA_ATTN_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return PELICA_ATTN_OK;
}

// One round of a prompt's keys (pelica_attn_prefill_round): key positions
// [key_begin, key_end) in rows from row 0, folded into state
struct Round {
    int32_t key_begin, key_end;
    float* state;
    int32_t first;
};

// prefill over the whole cache (round == NULL) or one round of keys; f32:
// f32 queries and output, else f16
int run_prefill(const PelicaAttnDesc* desc, const void* q, const uint16_t* k, const uint16_t* v, const float* sinks,
                void* out, bool f32, const Round* round, void* stream) {
    g_err[0] = 0;
    int rc = check_desc(desc);
    if (rc) return rc;
    const int es = f32 ? 4 : 2;
    rc = check_strides(desc, es, es);
    if (rc) return rc;
    if (desc->flags) return fail(PELICA_ATTN_EINVAL, "flags must be 0");
    if (round) {
        if (desc->n_seq != 1 || desc->ring_cap || desc->seq_kv_len)
            return fail(PELICA_ATTN_EINVAL, "rounds take one sequence of a linear cache");
        if (!q || !k || !v || !round->state)
            return fail(PELICA_ATTN_EINVAL, "q, k_rows, v_rows and state must be non-NULL");
        if (reinterpret_cast<uintptr_t>(round->state) % 4) return fail(PELICA_ATTN_EINVAL, "state must be 4-byte aligned");
        if (round->key_begin < 0 || round->key_end <= round->key_begin || round->key_end > desc->kv_len)
            return fail(PELICA_ATTN_EINVAL, "round [%d, %d) outside the %d keys", round->key_begin, round->key_end,
                        desc->kv_len);
    } else if (!q || !k || !v || !out) {
        return fail(PELICA_ATTN_EINVAL, "q, k, v and out must be non-NULL");
    }
    if (misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out))
        return fail(PELICA_ATTN_EINVAL, "q, k, v and out must be 16-byte aligned");
    pelica::PrefillParams p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.sinks = sinks;
    p.out = out;
    p.f32 = f32;
    p.q_tok = q_stride(desc);
    p.o_tok = o_stride(desc);
    p.seq_len = round ? nullptr : desc->seq_kv_len;
    p.seq_off = round ? nullptr : desc->seq_kv_offset;
    p.row_stride = desc->kv_row_stride ? desc->kv_row_stride : (int64_t)desc->n_kv * desc->hd;
    p.kv_len = desc->kv_len;
    p.n_head = desc->n_head;
    p.n_kv = desc->n_kv;
    p.hd = desc->hd;
    p.hpk = desc->n_head / desc->n_kv;
    p.T = desc->q_tokens;
    p.n_seq = desc->n_seq;
    p.window = desc->window;
    p.ring_cap = round ? 0 : desc->ring_cap;
    p.qscale = eff_scale(desc) * pelica::kLog2e;
    if (round) {
        p.key_begin = round->key_begin;
        p.key_end = round->key_end;
        p.first = round->first ? 1 : 0;
        p.state = round->state;
    }
    hipError_t e = pelica::launch_prefill(p, static_cast<hipStream_t>(stream));
    if (e == hipErrorNotSupported) return fail(PELICA_ATTN_EUNSUPPORTED, "prefill shape unsupported");
    if (e != hipSuccess) return fail(PELICA_ATTN_EHIP, "prefill launch: %s", hipGetErrorString(e));
    return PELICA_ATTN_OK;
}

}  // namespace

extern "C" {

int pelica_attn_decode_noalloc(const PelicaAttnDesc* desc, const float* q, const uint16_t* k, const uint16_t* v,
                               const float* sinks, float* out, void* stream) {
    g_err[0] = 0;
    DecodePlan pl;
    int rc = plan_decode(desc, &pl);
    if (rc) return rc;
    if (desc->flags) return fail(PELICA_ATTN_EINVAL, "flags must be 0");
    if (pl.ws_bytes > PELICA_ATTN_NOALLOC_SCRATCH_BYTES)
        return fail(PELICA_ATTN_EWORKSPACE, "this pass needs %zu bytes of scratch, above the %zu of the no-allocation "
                    "entry point (use pelica_attn_decode with a workspace)", pl.ws_bytes,
                    (size_t)PELICA_ATTN_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (pl.ws_bytes) {
        rc = scratch_of_current_device(&ws);
        if (rc) return rc;
    }
    return run_decode(desc, q, k, v, sinks, out, nullptr, ws, pl.ws_bytes ? PELICA_ATTN_NOALLOC_SCRATCH_BYTES : 0,
                      stream);
}

int pelica_attn_decode(const PelicaAttnDesc* desc, const float* q, const uint16_t* k, const uint16_t* v,
                       const float* sinks, float* out, void* workspace, size_t workspace_bytes, void* stream) {
    return run_decode(desc, q, k, v, sinks, out, nullptr, workspace, workspace_bytes, stream);
}

int pelica_attn_decode_partials(const PelicaAttnDesc* desc, const float* q, const uint16_t* k,
                                const uint16_t* v, float* parts, void* workspace, size_t workspace_bytes,
                                void* stream) {
    if (!parts) {
        g_err[0] = 0;
        return fail(PELICA_ATTN_EINVAL, "parts must be non-NULL");
    }
    return run_decode(desc, q, k, v, nullptr, nullptr, parts, workspace, workspace_bytes, stream);
}

int pelica_attn_decode_partials_range(const PelicaAttnDesc* desc, const float* q, const uint16_t* k_rows,
                                      const uint16_t* v_rows, int32_t key_begin, int32_t key_end, float* parts,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    if (!desc) return fail(PELICA_ATTN_EINVAL, "desc is NULL");
    if (!parts) return fail(PELICA_ATTN_EINVAL, "parts must be non-NULL");
    if (desc->n_seq != 1 || desc->seq_kv_len || desc->seq_kv_offset || desc->ring_cap)
        return fail(PELICA_ATTN_EINVAL, "a key range takes one sequence of a linear cache (n_seq 1, no seq_kv_len / "
                    "seq_kv_offset, ring_cap 0)");
    if (key_begin < 0 || key_end <= key_begin || key_end > desc->kv_len)
        return fail(PELICA_ATTN_EINVAL, "key range [%d, %d) outside the %d keys", key_begin, key_end, desc->kv_len);
    return run_decode(desc, q, k_rows, v_rows, nullptr, nullptr, parts, workspace, workspace_bytes, stream, key_begin,
                      key_end);
}

int pelica_attn_qkv_rope_cache(const PelicaAttnDesc* desc, const PelicaRope* rope, float* q, const float* k,
                               const float* v, int64_t token_stride, const float* q_norm, const float* k_norm,
                               float eps, uint16_t* k_cache, uint16_t* v_cache, void* stream) {
    g_err[0] = 0;
    if (!desc) return fail(PELICA_ATTN_EINVAL, "desc is NULL");
    const PelicaAttnDesc* d = desc;
    if (d->hd != 64 && d->hd != 128 && d->hd != 256) return fail(PELICA_ATTN_EUNSUPPORTED, "hd %d (64, 128 or 256)", d->hd);
    if (d->n_head <= 0 || d->n_kv <= 0 || d->n_head % d->n_kv) return fail(PELICA_ATTN_EINVAL, "bad head counts");
    if (d->n_seq <= 0 || d->q_tokens <= 0 || d->q_tokens > 65535 || d->n_seq > 65535)
        return fail(PELICA_ATTN_EINVAL, "n_seq and q_tokens must be in [1, 65535]");
    if (d->kv_len < d->q_tokens) return fail(PELICA_ATTN_EINVAL, "kv_len %d < q_tokens %d", d->kv_len, d->q_tokens);
    if ((d->seq_kv_len == nullptr) != (d->seq_kv_offset == nullptr) && d->seq_kv_len)
        return fail(PELICA_ATTN_EINVAL, "seq_kv_len needs seq_kv_offset");
    if (d->ring_cap < 0 || (d->ring_cap && d->ring_cap < d->q_tokens))
        return fail(PELICA_ATTN_EINVAL, "ring_cap %d cannot hold the pass's %d rows", d->ring_cap, d->q_tokens);
    if (d->flags) return fail(PELICA_ATTN_EINVAL, "flags must be 0");
    if (!q || !k || !v || !k_cache || !v_cache) return fail(PELICA_ATTN_EINVAL, "q, k, v and the caches must be non-NULL");
    const int64_t stride = d->kv_row_stride ? d->kv_row_stride : (int64_t)d->n_kv * d->hd;
    if (stride < (int64_t)d->n_kv * d->hd) return fail(PELICA_ATTN_EINVAL, "kv_row_stride below n_kv * hd");
    const int64_t tq = token_stride ? token_stride : (int64_t)d->n_head * d->hd;
    const int64_t tkv = token_stride ? token_stride : (int64_t)d->n_kv * d->hd;
    if (token_stride && token_stride < (int64_t)d->n_kv * d->hd)
        return fail(PELICA_ATTN_EINVAL, "token_stride below a token's heads");
    if (!(eps >= 0.f)) return fail(PELICA_ATTN_EINVAL, "eps must be >= 0");
    pelica::QkvParams p{};
    if (rope && rope->rot) {
        if (rope->rot < 0 || rope->rot % 2 || rope->rot > d->hd) return fail(PELICA_ATTN_EINVAL, "rot %d", rope->rot);
        if (!rope->table || rope->table_split < 0) return fail(PELICA_ATTN_EINVAL, "rope table missing");
        if (rope->table_split && rope->table_rows < rope->table_split + 256)
            return fail(PELICA_ATTN_EINVAL, "a two-level rope table needs %d rows", rope->table_split + 256);
        const long long covered = rope->table_split ? 256LL * rope->table_split : rope->table_rows;
        if (covered < d->kv_len)
            return fail(PELICA_ATTN_EINVAL, "rope table covers %lld positions, kv_len is %d", covered, d->kv_len);
        p.table = rope->table;
        p.rot = rope->rot;
        p.neox = rope->neox ? 1 : 0;
        p.table_split = rope->table_split;
    }
    p.q = q;
    p.k = k;
    p.v = v;
    p.tok_q = tq;
    p.tok_kv = tkv;
    p.q_norm = q_norm;
    p.k_norm = k_norm;
    p.eps = eps;
    p.k_cache = k_cache;
    p.v_cache = v_cache;
    p.seq_len = d->seq_kv_len;
    p.seq_off = d->seq_kv_offset;
    p.row_stride = stride;
    p.kv_len = d->kv_len;
    p.n_head = d->n_head;
    p.n_kv = d->n_kv;
    p.hd = d->hd;
    p.T = d->q_tokens;
    p.n_seq = d->n_seq;
    p.ring_cap = d->ring_cap;
    hipError_t e = pelica::launch_qkv(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(PELICA_ATTN_EHIP, "qkv launch: %s", hipGetErrorString(e));
    return PELICA_ATTN_OK;
}

size_t pelica_attn_mla_workspace_bytes(const PelicaAttnDesc* desc) {
    g_err[0] = 0;
    DecodePlan pl;
    if (plan_mla(desc, &pl)) return 0;
    return pl.ws_bytes;
}

int pelica_attn_mla(const PelicaAttnDesc* desc, const float* q, const uint16_t* latent, float* out, void* workspace,
                    size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    DecodePlan pl;
    int rc = plan_mla(desc, &pl);
    if (rc) return rc;
    rc = check_strides(desc, 4, 4);
    if (rc) return rc;
    if (desc->flags) return fail(PELICA_ATTN_EINVAL, "flags must be 0");
    if (!q || !latent || !out) return fail(PELICA_ATTN_EINVAL, "q, latent and out must be non-NULL");
    if (misaligned(q) || misaligned(latent) || misaligned(out) || misaligned(workspace))
        return fail(PELICA_ATTN_EINVAL, "q, latent, out and workspace must be 16-byte aligned");
    if (pl.ws_bytes && (!workspace || workspace_bytes < pl.ws_bytes))
        return fail(PELICA_ATTN_EWORKSPACE, "workspace of %zu bytes needed, %zu given", pl.ws_bytes,
                    workspace ? workspace_bytes : (size_t)0);
    pelica::DecodeParams p{};
    p.q = q;
    p.k = latent;
    p.v = latent;
    p.out = out;
    char* ws = static_cast<char*>(workspace);
    p.ws_ml = pl.ws_bytes ? reinterpret_cast<float*>(ws) : nullptr;
    p.ws_o = pl.ws_bytes ? reinterpret_cast<float*>(ws + pl.ml_bytes) : nullptr;
    p.seq_len = desc->seq_kv_len;
    p.seq_off = desc->seq_kv_offset;
    p.row_stride = desc->kv_row_stride ? desc->kv_row_stride : 512;
    p.q_tok = q_stride(desc);
    p.o_tok = o_stride(desc);
    p.kr_lo = 0;
    p.kr_hi = INT32_MAX;
    p.kv_len = desc->kv_len;
    p.n_head = desc->n_head;
    p.n_kv = 1;
    p.hd = 512;
    p.hpk = desc->n_head;
    p.T = desc->q_tokens;
    p.R = pl.R;
    p.n_rg = pl.n_rg;
    p.n_seq = desc->n_seq;
    p.qscale = eff_scale(desc) * pelica::kLog2e;
    p.n_slot = pl.n_slot;
    p.split_keys = pl.split_keys;
    p.wg_heads = 1;
    p.rg_rows = 16 * pl.rt;
    hipError_t e = pelica::launch_mla(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(PELICA_ATTN_EHIP, "mla launch: %s", hipGetErrorString(e));
    return PELICA_ATTN_OK;
}

int pelica_attn_prefill(const PelicaAttnDesc* desc, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        const float* sinks, uint16_t* out, void* stream) {
    return run_prefill(desc, q, k, v, sinks, out, false, nullptr, stream);
}

int pelica_attn_prefill_f32(const PelicaAttnDesc* desc, const float* q, const uint16_t* k, const uint16_t* v,
                            const float* sinks, float* out, void* stream) {
    return run_prefill(desc, q, k, v, sinks, out, true, nullptr, stream);
}

int pelica_attn_prefill_round(const PelicaAttnDesc* desc, const uint16_t* q, const uint16_t* k_rows,
                              const uint16_t* v_rows, int32_t key_begin, int32_t key_end, const float* sinks,
                              float* state, int32_t first, uint16_t* out, void* stream) {
    const Round r{key_begin, key_end, state, first};
    return run_prefill(desc, q, k_rows, v_rows, sinks, out, false, &r, stream);
}

int pelica_attn_prefill_round_f32(const PelicaAttnDesc* desc, const float* q, const uint16_t* k_rows,
                                  const uint16_t* v_rows, int32_t key_begin, int32_t key_end, const float* sinks,
                                  float* state, int32_t first, float* out, void* stream) {
    const Round r{key_begin, key_end, state, first};
    return run_prefill(desc, q, k_rows, v_rows, sinks, out, true, &r, stream);
}

int pelica_attn_partials_merge_batch(int32_t n_tokens, int32_t n_head, int32_t hd, int32_t n_parts,
                                     const float* parts, const float* sinks, float* out, void* stream) {
    g_err[0] = 0;
    if (n_tokens <= 0 || n_tokens > 65535 || n_head <= 0 || n_parts <= 0)
        return fail(PELICA_ATTN_EINVAL, "n_tokens %d (<= 65535), n_head %d and n_parts %d must be positive", n_tokens,
                    n_head, n_parts);
    if (hd <= 0 || hd % 2 || hd > 1024) return fail(PELICA_ATTN_EINVAL, "hd %d must be even, in [2, 1024]", hd);
    if (!parts || !out) return fail(PELICA_ATTN_EINVAL, "parts and out must be non-NULL");
    if (reinterpret_cast<uintptr_t>(parts) % 8 || reinterpret_cast<uintptr_t>(out) % 8)
        return fail(PELICA_ATTN_EINVAL, "parts and out must be 8-byte aligned");
    hipError_t e = pelica::launch_partials_merge(n_tokens, n_head, hd, n_parts, parts, sinks, out,
                                                 static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(PELICA_ATTN_EHIP, "merge launch: %s", hipGetErrorString(e));
    return PELICA_ATTN_OK;
}

int pelica_attn_partials_merge(int32_t n_head, int32_t hd, int32_t n_parts, const float* parts, const float* sinks,
                               float* out, void* stream) {
    return pelica_attn_partials_merge_batch(1, n_head, hd, n_parts, parts, sinks, out, stream);
}

}  // extern "C"
