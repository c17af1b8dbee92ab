/* CPU oracle of the step before attention — TEST INFRASTRUCTURE ONLY (see
 * attn_oracle.h): per-head RMS norm, rotary embedding and the f16 cache
 * write of the new K/V rows, restating qk_dec (src/moe_kernels.rs:304-378)
 * and ROPE_KV_T (src/oss_batch.rs:113-170).  Plain C, no contraction
 * (-ffp-contract=off): every product and sum rounds as written. */
#include <math.h>

#include "attn_oracle.h"

/* cos, sin of rotary pair j at position pos (src/moe_kernels.rs:350-355 for
 * the two-level table, src/oss_batch.rs:151-152 for the direct one) */
static void rope_cs(const OrcRope* r, int pos, int j, float* cs, float* sn) {
    const int half = r->rot / 2;
    if (r->table_split <= 0) {
        *cs = r->table[((size_t)pos * half + j) * 2];
        *sn = r->table[((size_t)pos * half + j) * 2 + 1];
        return;
    }
    const float* hi = r->table + ((size_t)(pos / 256) * half + j) * 2;
    const float* lo = r->table + ((size_t)(r->table_split + pos % 256) * half + j) * 2;
    const float c1 = hi[0], s1 = hi[1], c2 = lo[0], s2 = lo[1];
    const float a = c1 * c2, b = s1 * s2, c = s1 * c2, e = c1 * s2;
    *cs = a - b;
    *sn = c + e;
}

/* one head in place: RMS norm (w != NULL), then rope (r != NULL) */
static void head_norm_rope(float* x, int hd, const float* w, float eps, const OrcRope* r, int pos) {
    if (w) {
        float tot = 0.f;
        for (int i = 0; i < hd; ++i) {
            const float sq = x[i] * x[i];
            tot += sq;
        }
        const float inv = 1.f / sqrtf(tot / (float)hd + eps);
        for (int i = 0; i < hd; ++i) {
            const float y = x[i] * inv;
            x[i] = y * w[i];
        }
    }
    if (r) {
        const int half = r->rot / 2;
        for (int j = 0; j < half; ++j) {
            const int a = r->neox ? j : 2 * j, b = r->neox ? j + half : 2 * j + 1;
            float cs, sn;
            rope_cs(r, pos, j, &cs, &sn);
            const float x0 = x[a], x1 = x[b];
            const float p0 = x0 * cs, p1 = x1 * sn, p2 = x0 * sn, p3 = x1 * cs;
            x[a] = p0 - p1;
            x[b] = p2 + p3;
        }
    }
}

int orc_qk_norm_rope_cache(const OrcDesc* d, const OrcRope* r, float* q, const float* k, const float* v,
                           const float* q_norm, const float* k_norm, float eps,
                           uint16_t* k_cache, uint16_t* v_cache) {
    const int hd = d->hd, T = d->q_tokens;
    if (hd <= 0 || hd > 1024 || d->n_head <= 0 || d->n_kv <= 0 || T <= 0 || d->n_seq <= 0) return -1;
    if (r && (r->rot <= 0 || r->rot > hd || r->rot % 2 || !r->table)) return -1;
    const int64_t stride = d->kv_row_stride ? d->kv_row_stride : (int64_t)d->n_kv * hd;
    float buf[1024];
    for (int s = 0; s < d->n_seq; ++s) {
        const int len = d->seq_kv_len[s];
        if (len < T) return -1;
        for (int t = 0; t < T; ++t) {
            const int pos = len - T + t;
            const int64_t row = d->seq_kv_off[s] + (d->ring_cap ? pos % d->ring_cap : pos);
            for (int h = 0; h < d->n_head; ++h)
                head_norm_rope(q + (((size_t)s * T + t) * d->n_head + h) * hd, hd, q_norm, eps, r, pos);
            for (int h = 0; h < d->n_kv; ++h) {
                const size_t src = (((size_t)s * T + t) * d->n_kv + h) * hd;
                for (int i = 0; i < hd; ++i) buf[i] = k[src + i];
                head_norm_rope(buf, hd, k_norm, eps, r, pos);
                for (int i = 0; i < hd; ++i) {
                    k_cache[row * stride + (int64_t)h * hd + i] = orc_f32_to_f16(buf[i]);
                    v_cache[row * stride + (int64_t)h * hd + i] = orc_f32_to_f16(v[src + i]);
                }
            }
        }
    }
    return 0;
}
