/* CPU oracle for Pelica's attention path — TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference's CPU decode attention (src/cpu_attn.rs) so that
 * the HIP kernels of libpelica_attn.so can be checked against the same
 * arithmetic, and adds the chunk combine, sinks, windows, drafts and ring
 * addressing of the GPU call sites (citations per function).  Built with
 * -ffp-contract=off: every fma below is explicit, every other product and
 * sum rounds on its own, as in the Rust code (Rust never contracts).
 *
 * Parity pins (tests/test_oracle.py): closed forms (equal keys, single key,
 * sink identity, window >= context), an fp64 brute force on small shapes,
 * split/order independence of the merge, and bitwise agreement of the
 * AVX2 and scalar chunk paths (the reference's own check_attn pin,
 * src/moe.rs:1909-1913).  Bitwise identity with the Rust binary itself is
 * "parity unpinned" (no Rust toolchain here); the tolerance contract does
 * not need it.
 */
#include "attn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* src/moe_kernels.rs:437-444 (Cephes expf constants). */
static const float K_LOG2E = 1.44269504f;
static const float K_C1 = 0.693359375f;
static const float K_C2 = -2.12194440e-4f;
static const float K_P[6] = {1.98756915e-4f, 1.39819995e-3f, 8.3334519e-3f,
                             4.1665796e-2f, 0.16666665f, 0.50000001f};
static const float K_MIN = -40.0f;
/* the "empty" max of the running states (src/cpu_attn.rs:90) */
static const float NEG_BIG = -3.0e38f;

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* src/cpu_attn.rs:28-44 */
float orc_pexp(float x) {
    if (x < K_MIN) return 0.0f;
    float n = floorf(fmaf(x, K_LOG2E, 0.5f));
    float r = fmaf(n, -K_C1, x);
    r = fmaf(n, -K_C2, r);
    float p = K_P[0];
    for (int i = 1; i < 6; ++i) p = fmaf(p, r, K_P[i]);
    float y = fmaf(p, r * r, r);
    y = y + 1.0f;
    return y * bits_f32((uint32_t)((int32_t)n + 127) << 23);
}

/* src/cpu_attn.rs:46-66 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t s = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {
            uint32_t ee = 113;
            while ((m & 0x400u) == 0) { m <<= 1; --ee; }
            bits = s | (ee << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    return bits_f32(bits);
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) /* rounds to >= 65520: overflow */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* below the smallest normal half: subnormal or 0 */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* value = m * 2^(e-150); half unit 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - 0x38000000u; /* rebias exponent 127 -> 15 */
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) ++q;
    return (uint16_t)(sign | q);
}

/* ---- one chunk: src/cpu_attn.rs:81-216 ---------------------------------- */

typedef struct {
    float *m, *l, *o; /* per (stream, head): 4*nh, 4*nh, 4*nh*hd */
} Streams;

static int streams_init(Streams* st, int nh, int hd) {
    st->m = (float*)malloc(sizeof(float) * 4 * nh);
    st->l = (float*)calloc(4 * (size_t)nh, sizeof(float));
    st->o = (float*)calloc(4 * (size_t)nh * hd, sizeof(float));
    if (!st->m || !st->l || !st->o) return -1;
    for (int i = 0; i < 4 * nh; ++i) st->m[i] = NEG_BIG;
    return 0;
}

static void streams_free(Streams* st) { free(st->m); free(st->l); free(st->o); }

/* the 4-stream merge of src/cpu_attn.rs:93-115 */
static void streams_finish(const Streams* st, int nh, int hd, float* out) {
    for (int h = 0; h < nh; ++h) {
        int s[4] = {h, nh + h, 2 * nh + h, 3 * nh + h};
        float m[4], w[4];
        for (int t = 0; t < 4; ++t) m[t] = st->m[s[t]];
        float mx = fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3]));
        for (int t = 0; t < 4; ++t) w[t] = orc_pexp(m[t] - mx);
        float* ob = out + (size_t)h * (hd + 2);
        ob[0] = mx;
        float l = st->l[s[0]] * w[0];
        for (int t = 1; t < 4; ++t) l = fmaf(st->l[s[t]], w[t], l);
        ob[1] = l;
        for (int i = 0; i < hd; ++i) {
            float o = st->o[(size_t)s[0] * hd + i] * w[0];
            for (int t = 1; t < 4; ++t) o = fmaf(st->o[(size_t)s[t] * hd + i], w[t], o);
            ob[2 + i] = o;
        }
    }
}

/* online-softmax update of one (stream, head) with score x (src/cpu_attn.rs:148-157) */
static inline void stream_update(Streams* st, int s, int hd, float x, const float* vf) {
    float mn = fmaxf(st->m[s], x);
    float c = orc_pexp(st->m[s] - mn);
    float p = orc_pexp(x - mn);
    st->l[s] = fmaf(st->l[s], c, p);
    float* o = st->o + (size_t)s * hd;
    for (int i = 0; i < hd; ++i) o[i] = fmaf(o[i], c, p * vf[i]);
    st->m[s] = mn;
}

/* src/cpu_attn.rs:118-162 */
void orc_chunk_scalar(int hd, int n_kv, int hpk, int kv0, int kv1, int n,
                      const uint16_t* k, const uint16_t* v, const float* q, float* out) {
    const int rl = n_kv * hd, nh = (kv1 - kv0) * hpk, d = hd / 32;
    Streams st;
    if (streams_init(&st, nh, hd)) abort();
    float* kf = (float*)malloc(sizeof(float) * hd);
    float* vf = (float*)malloc(sizeof(float) * hd);
    for (int j = 0; j < n; ++j) {
        int sg = j % 4;
        for (int g = kv0; g < kv1; ++g) {
            size_t at = (size_t)j * rl + (size_t)g * hd;
            for (int i = 0; i < hd; ++i) {
                kf[i] = orc_f16_to_f32(k[at + i]);
                vf[i] = orc_f16_to_f32(v[at + i]);
            }
            for (int hh = (g - kv0) * hpk; hh < (g + 1 - kv0) * hpk; ++hh) {
                const float* qh = q + (size_t)hh * hd;
                float x[32];
                /* lane i: dims i, i+32, ... in order, fmas after the first product */
                for (int lane = 0; lane < 32; ++lane) {
                    float a = qh[lane] * kf[lane];
                    for (int i = 1; i < d; ++i) a = fmaf(qh[lane + 32 * i], kf[lane + 32 * i], a);
                    x[lane] = a;
                }
                /* xor-shuffle reduction order 16, 8, 4, 2, 1 */
                for (int off = 16; off >= 1; off >>= 1)
                    for (int i = 0; i < off; ++i) x[i] = x[i] + x[i + off];
                stream_update(&st, sg * nh + hh, hd, x[0], vf);
            }
        }
    }
    streams_finish(&st, nh, hd, out);
    free(kf); free(vf);
    streams_free(&st);
}

#if defined(__x86_64__)
/* src/cpu_attn.rs:164-216: the same lanes as orc_chunk_scalar, 8 per ymm. */
__attribute__((target("avx2,fma,f16c")))
static void chunk_avx2_impl(int hd, int n_kv, int hpk, int kv0, int kv1, int n,
                            const uint16_t* k, const uint16_t* v, const float* q, float* out) {
    const int rl = n_kv * hd, nh = (kv1 - kv0) * hpk, d = hd / 32, nb = hd / 8;
    Streams st;
    if (streams_init(&st, nh, hd)) abort();
    float* kf = (float*)aligned_alloc(32, sizeof(float) * (size_t)(hd < 8 ? 8 : hd));
    float* vf = (float*)aligned_alloc(32, sizeof(float) * (size_t)(hd < 8 ? 8 : hd));
    for (int j = 0; j < n; ++j) {
        int sg = j % 4;
        for (int g = kv0; g < kv1; ++g) {
            size_t at = (size_t)j * rl + (size_t)g * hd;
            for (int b = 0; b < nb; ++b) {
                _mm256_store_ps(kf + 8 * b, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(k + at + 8 * b))));
                _mm256_store_ps(vf + 8 * b, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(v + at + 8 * b))));
            }
            for (int hh = (g - kv0) * hpk; hh < (g + 1 - kv0) * hpk; ++hh) {
                const float* qh = q + (size_t)hh * hd;
                __m256 x[4];
                for (int b = 0; b < 4; ++b) {
                    __m256 a = _mm256_mul_ps(_mm256_loadu_ps(qh + 8 * b), _mm256_load_ps(kf + 8 * b));
                    for (int i = 1; i < d; ++i)
                        a = _mm256_fmadd_ps(_mm256_loadu_ps(qh + 32 * i + 8 * b), _mm256_load_ps(kf + 32 * i + 8 * b), a);
                    x[b] = a;
                }
                /* xor 16 then 8: (x0+x2)+(x1+x3); then 4, 2, 1 inside the register */
                __m256 s8 = _mm256_add_ps(_mm256_add_ps(x[0], x[2]), _mm256_add_ps(x[1], x[3]));
                __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(s8), _mm256_extractf128_ps(s8, 1));
                __m128 s2 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));
                float sc = _mm_cvtss_f32(_mm_add_ss(s2, _mm_shuffle_ps(s2, s2, 1)));
                int s = sg * nh + hh;
                float mn = fmaxf(st.m[s], sc);
                float c = orc_pexp(st.m[s] - mn);
                float p = orc_pexp(sc - mn);
                st.l[s] = fmaf(st.l[s], c, p);
                __m256 cv = _mm256_set1_ps(c), pv = _mm256_set1_ps(p);
                float* o = st.o + (size_t)s * hd;
                for (int b = 0; b < nb; ++b) {
                    __m256 ov = _mm256_loadu_ps(o + 8 * b);
                    _mm256_storeu_ps(o + 8 * b, _mm256_fmadd_ps(ov, cv, _mm256_mul_ps(pv, _mm256_load_ps(vf + 8 * b))));
                }
                st.m[s] = mn;
            }
        }
    }
    streams_finish(&st, nh, hd, out);
    free(kf); free(vf);
    streams_free(&st);
}
#endif

static int have_avx2(void) {
#if defined(__x86_64__)
    static int cached = -1;
    if (cached < 0) {
        __builtin_cpu_init();
        cached = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
    }
    return cached;
#else
    return 0;
#endif
}

int orc_chunk_avx2(int hd, int n_kv, int hpk, int kv0, int kv1, int n,
                   const uint16_t* k, const uint16_t* v, const float* q, float* out) {
#if defined(__x86_64__)
    if (!have_avx2()) return 0;
    chunk_avx2_impl(hd, n_kv, hpk, kv0, kv1, n, k, v, q, out);
    return 1;
#else
    (void)hd; (void)n_kv; (void)hpk; (void)kv0; (void)kv1; (void)n; (void)k; (void)v; (void)q; (void)out;
    return 0;
#endif
}

/* src/cpu_attn.rs:72-79 */
void orc_chunk(int hd, int n_kv, int hpk, int kv0, int kv1, int n,
               const uint16_t* k, const uint16_t* v, const float* q, float* out) {
    if (orc_chunk_avx2(hd, n_kv, hpk, kv0, kv1, n, k, v, q, out)) return;
    orc_chunk_scalar(hd, n_kv, hpk, kv0, kv1, n, k, v, q, out);
}

/* ---- combine: src/moe_kernels.rs:585-617 with the sink of
 *      src/oss_batch.rs:395-425 (the sink joins the max and adds
 *      e^{sink-M} to the denominator).  The reference's merge uses the
 *      GPU's exp; the oracle uses pexp (the same function to ~1 ulp). ---- */
void orc_merge_head(int hd, int n_parts, const float* parts, size_t part_stride,
                    const float* sink, float* out) {
    float M = sink ? *sink : NEG_BIG;
    for (int c = 0; c < n_parts; ++c) M = fmaxf(M, parts[(size_t)c * part_stride]);
    float L = sink ? orc_pexp(*sink - M) : 0.0f;
    for (int i = 0; i < hd; ++i) out[i] = 0.0f;
    for (int c = 0; c < n_parts; ++c) {
        const float* p = parts + (size_t)c * part_stride;
        float w = orc_pexp(p[0] - M);
        L = fmaf(p[1], w, L);
        for (int i = 0; i < hd; ++i) out[i] = fmaf(p[2 + i], w, out[i]);
    }
    for (int i = 0; i < hd; ++i) out[i] = out[i] / L;
}

/* ---- whole attention ---------------------------------------------------- */

static int desc_ok(const OrcDesc* d) {
    if (!d || d->n_head <= 0 || d->n_kv <= 0 || d->hd <= 0 || d->hd % 32) return 0;
    if (d->n_head % d->n_kv || d->n_seq <= 0 || d->q_tokens <= 0) return 0;
    if (!d->seq_kv_len || d->kv_row_stride < (int64_t)d->n_kv * d->hd) return 0;
    if (d->window < 0 || d->ring_cap < 0) return 0;
    for (int s = 0; s < d->n_seq; ++s) {
        int len = d->seq_kv_len[s];
        if (len < d->q_tokens) return 0;
        if (d->ring_cap) {
            /* every key some token of the pass sees must still be in the ring */
            int pos0 = len - d->q_tokens, lo0 = 0;
            if (d->window > 0 && pos0 + 1 > d->window) lo0 = pos0 + 1 - d->window;
            if (len - lo0 > d->ring_cap) return 0;
        }
    }
    return 1;
}

static inline int64_t seq_row0(const OrcDesc* d, int s) {
    if (d->seq_kv_off) return d->seq_kv_off[s];
    int64_t r = 0;
    for (int i = 0; i < s; ++i) r += d->seq_kv_len[i];
    return r;
}

/* Gather rows [a, b) of sequence s (ring or linear) into contiguous
 * n_kv*hd rows, as the chunk routine expects them. */
static void gather_rows(const OrcDesc* d, int s, int64_t row0, int a, int b,
                        const uint16_t* src, uint16_t* dst) {
    const size_t rl = (size_t)d->n_kv * d->hd;
    (void)s;
    for (int j = a; j < b; ++j) {
        int64_t r = d->ring_cap ? (int64_t)(j % d->ring_cap) : (int64_t)j;
        memcpy(dst + (size_t)(j - a) * rl, src + (size_t)(row0 + r) * d->kv_row_stride, rl * 2);
    }
}

static inline void key_range(const OrcDesc* d, int len, int t, int* lo, int* pos) {
    int p = len - d->q_tokens + t;
    int l = 0;
    if (d->window > 0 && p + 1 > d->window) l = p + 1 - d->window;
    *lo = l;
    *pos = p;
}

/* Partials of chunk c (positions [c*256, c*256+256) clipped to [lo, pos]) of
 * one token for kv heads [kv0, kv1). */
static void token_chunk(const OrcDesc* d, const float* qs, const uint16_t* k, const uint16_t* v,
                        int s, int64_t row0, int lo, int pos, int c, int kv0, int kv1,
                        uint16_t* kb, uint16_t* vb, float* out) {
    int a = c * ORC_CHUNK, b = a + ORC_CHUNK;
    if (a < lo) a = lo;
    if (b > pos + 1) b = pos + 1;
    gather_rows(d, s, row0, a, b, k, kb);
    gather_rows(d, s, row0, a, b, v, vb);
    const int hpk = d->n_head / d->n_kv;
    orc_chunk(d->hd, d->n_kv, hpk, kv0, kv1, b - a, kb, vb, qs + (size_t)kv0 * hpk * d->hd, out);
}

static int n_threads(int threads) {
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

int orc_attn(const OrcDesc* d, const float* q, const uint16_t* k, const uint16_t* v,
             const float* sinks, float* out, int t_begin, int t_end, int threads) {
    if (!desc_ok(d)) return -1;
    if (t_begin < 0) t_begin = 0;
    if (t_end > d->q_tokens || t_end < 0) t_end = d->q_tokens;
    const int nh = d->n_head, hd = d->hd, hp = hd + 2;
    const size_t rl = (size_t)d->n_kv * hd;
    const int nt = n_threads(threads);
    const int T = t_end - t_begin;
    if (T <= 0) return 0;
    const int ntask = d->n_seq * T;
    int64_t* row0 = (int64_t*)malloc(sizeof(int64_t) * d->n_seq);
    for (int s = 0; s < d->n_seq; ++s) row0[s] = seq_row0(d, s);

    if (ntask >= 2 * nt) {
        /* many tokens: one task per (sequence, token), chunks in order */
#pragma omp parallel num_threads(nt)
        {
            uint16_t* kb = (uint16_t*)malloc(rl * ORC_CHUNK * 2);
            uint16_t* vb = (uint16_t*)malloc(rl * ORC_CHUNK * 2);
            float* qs = (float*)malloc(sizeof(float) * nh * hd);
            int maxc = 0;
            for (int s = 0; s < d->n_seq; ++s)
                if (d->seq_kv_len[s] / ORC_CHUNK + 1 > maxc) maxc = d->seq_kv_len[s] / ORC_CHUNK + 1;
            float* parts = (float*)malloc(sizeof(float) * (size_t)maxc * nh * hp);
#pragma omp for schedule(dynamic, 1)
            for (int task = 0; task < ntask; ++task) {
                int s = task / T, t = t_begin + task % T;
                int lo, pos;
                key_range(d, d->seq_kv_len[s], t, &lo, &pos);
                const float* qt = q + ((size_t)s * d->q_tokens + t) * nh * hd;
                for (int i = 0; i < nh * hd; ++i) qs[i] = qt[i] * d->scale;
                int c0 = lo / ORC_CHUNK, c1 = pos / ORC_CHUNK;
                for (int c = c0; c <= c1; ++c)
                    token_chunk(d, qs, k, v, s, row0[s], lo, pos, c, 0, d->n_kv, kb, vb,
                                parts + (size_t)(c - c0) * nh * hp);
                float* ot = out + ((size_t)s * d->q_tokens + t) * nh * hd;
                for (int h = 0; h < nh; ++h)
                    orc_merge_head(hd, c1 - c0 + 1, parts + (size_t)h * hp, (size_t)nh * hp,
                                   sinks ? sinks + h : NULL, ot + (size_t)h * hd);
            }
            free(kb); free(vb); free(qs); free(parts);
        }
    } else {
        /* few tokens (decode): tasks = (chunk, kv-head group) per token, as
         * the reference's CPU tier splits them (src/moe.rs:1692-1712) */
        float* qs = (float*)malloc(sizeof(float) * nh * hd);
        for (int task = 0; task < ntask; ++task) {
            int s = task / T, t = t_begin + task % T;
            int lo, pos;
            key_range(d, d->seq_kv_len[s], t, &lo, &pos);
            const float* qt = q + ((size_t)s * d->q_tokens + t) * nh * hd;
            for (int i = 0; i < nh * hd; ++i) qs[i] = qt[i] * d->scale;
            int c0 = lo / ORC_CHUNK, c1 = pos / ORC_CHUNK, nc = c1 - c0 + 1;
            int ng = (2 * nt + nc - 1) / nc;
            if (ng < 1) ng = 1;
            if (ng > d->n_kv) ng = d->n_kv;
            float* parts = (float*)malloc(sizeof(float) * (size_t)nc * nh * hp);
            const int hpk = nh / d->n_kv;
#pragma omp parallel num_threads(nt)
            {
                uint16_t* kb = (uint16_t*)malloc(rl * ORC_CHUNK * 2);
                uint16_t* vb = (uint16_t*)malloc(rl * ORC_CHUNK * 2);
#pragma omp for schedule(dynamic, 1)
                for (int x = 0; x < nc * ng; ++x) {
                    int c = c0 + x / ng, gi = x % ng;
                    int kv0 = gi * d->n_kv / ng, kv1 = (gi + 1) * d->n_kv / ng;
                    token_chunk(d, qs, k, v, s, row0[s], lo, pos, c, kv0, kv1, kb, vb,
                                parts + (size_t)(c - c0) * nh * hp + (size_t)kv0 * hpk * hp);
                }
                free(kb); free(vb);
            }
            float* ot = out + ((size_t)s * d->q_tokens + t) * nh * hd;
            for (int h = 0; h < nh; ++h)
                orc_merge_head(hd, nc, parts + (size_t)h * hp, (size_t)nh * hp,
                               sinks ? sinks + h : NULL, ot + (size_t)h * hd);
            free(parts);
        }
        free(qs);
    }
    free(row0);
    return 0;
}

int orc_attn_f16(const OrcDesc* d, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                 const float* sinks, uint16_t* out, int t_begin, int t_end, int threads) {
    if (!desc_ok(d)) return -1;
    size_t n = (size_t)d->n_seq * d->q_tokens * d->n_head * d->hd;
    float* qf = (float*)malloc(sizeof(float) * n);
    float* of = (float*)calloc(n, sizeof(float));
    for (size_t i = 0; i < n; ++i) qf[i] = orc_f16_to_f32(q[i]);
    int rc = orc_attn(d, qf, k, v, sinks, of, t_begin, t_end, threads);
    if (rc == 0) {
        if (t_begin < 0) t_begin = 0;
        if (t_end > d->q_tokens || t_end < 0) t_end = d->q_tokens;
        const size_t per = (size_t)d->n_head * d->hd;
        for (int s = 0; s < d->n_seq; ++s)
            for (int t = t_begin; t < t_end; ++t) {
                size_t b = ((size_t)s * d->q_tokens + t) * per;
                for (size_t i = 0; i < per; ++i) out[b + i] = orc_f32_to_f16(of[b + i]);
            }
    }
    free(qf); free(of);
    return rc;
}

int orc_partials(const OrcDesc* d, const float* q, const uint16_t* k, const uint16_t* v,
                 int s, int t, int k_begin, int k_end, float* parts, int threads) {
    if (!desc_ok(d) || s < 0 || s >= d->n_seq || t < 0 || t >= d->q_tokens) return -1;
    const int nh = d->n_head, hd = d->hd, hp = hd + 2;
    int lo, pos;
    key_range(d, d->seq_kv_len[s], t, &lo, &pos);
    if (k_begin > lo) lo = k_begin;
    if (k_end - 1 < pos) pos = k_end - 1;
    if (pos < lo) return 0;
    float* qs = (float*)malloc(sizeof(float) * nh * hd);
    const float* qt = q + ((size_t)s * d->q_tokens + t) * nh * hd;
    for (int i = 0; i < nh * hd; ++i) qs[i] = qt[i] * d->scale;
    int c0 = lo / ORC_CHUNK, c1 = pos / ORC_CHUNK;
    int64_t r0 = seq_row0(d, s);
    const size_t rl = (size_t)d->n_kv * hd;
#pragma omp parallel num_threads(n_threads(threads))
    {
        uint16_t* kb = (uint16_t*)malloc(rl * ORC_CHUNK * 2);
        uint16_t* vb = (uint16_t*)malloc(rl * ORC_CHUNK * 2);
#pragma omp for schedule(dynamic, 1)
        for (int c = c0; c <= c1; ++c)
            token_chunk(d, qs, k, v, s, r0, lo, pos, c, 0, d->n_kv, kb, vb,
                        parts + (size_t)(c - c0) * nh * hp);
        free(kb); free(vb);
    }
    free(qs);
    return c1 - c0 + 1;
}
