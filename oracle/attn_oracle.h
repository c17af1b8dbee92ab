/* CPU oracle for Pelica's attention path — TEST INFRASTRUCTURE ONLY.
 *
 * A C restatement of the reference's CPU decode attention
 * (src/cpu_attn.rs) plus the pieces the GPU path adds around it: the
 * fixed-order combine of chunk partials (merge_dec, src/moe_kernels.rs:585-617),
 * learned sink logits (ATTN_M, src/oss_batch.rs:395-425), sliding windows and
 * causal drafts (ATTN_T, src/oss_batch.rs:172-251; attn_p,
 * src/oss_prefill.rs:391-526) and ring-buffer row addressing.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the CPU baseline. The
 * product path (pelica_amd, libpelica_attn.so) never links or calls it.
 */
#ifndef PELICA_ATTN_ORACLE_H
#define PELICA_ATTN_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Keys per CPU chunk (src/moe_kernels.rs:295, CHUNK = 256). */
#define ORC_CHUNK 256

/* Cephes expf restated with explicit fmas, e^x for x <= 0, 0 below -40
 * (src/cpu_attn.rs:28-44, constants src/moe_kernels.rs:437-444). */
float orc_pexp(float x);
/* IEEE half -> single including subnormals, inf and nan (src/cpu_attn.rs:46-66). */
float orc_f16_to_f32(uint16_t h);
/* single -> half, round to nearest even (test-input and f16-output helper). */
uint16_t orc_f32_to_f16(float f);

/* Partials (max, sum, hd sums of v) of one chunk of n <= 256 keys for the
 * query heads of kv heads [kv0, kv1): k, v are n rows of n_kv*hd f16, q holds
 * those heads' queries (hd each, already scaled), out gets
 * (kv1-kv0)*hpk*(hd+2) floats.  src/cpu_attn.rs:72-79 (dispatch),
 * :118-162 (scalar), :164-216 (AVX2+FMA+F16C). hd must be a multiple of 32. */
void orc_chunk(int hd, int n_kv, int hpk, int kv0, int kv1, int n,
               const uint16_t* k, const uint16_t* v, const float* q, float* out);
void orc_chunk_scalar(int hd, int n_kv, int hpk, int kv0, int kv1, int n,
                      const uint16_t* k, const uint16_t* v, const float* q, float* out);
/* returns 0 when the CPU lacks AVX2/FMA/F16C (nothing written) */
int orc_chunk_avx2(int hd, int n_kv, int hpk, int kv0, int kv1, int n,
                   const uint16_t* k, const uint16_t* v, const float* q, float* out);

/* Combine n_parts partials of one head, laid out with a stride of
 * part_stride floats (merge_dec's (c*n_head+h)*(hd+2) layout gives
 * part_stride = n_head*(hd+2)), in order, with an optional sink logit:
 * out[i] = sum_c O_c[i] w_c / (e^{sink-M} + sum_c L_c w_c), w_c = e^{M_c-M}.
 * src/moe_kernels.rs:585-617, src/oss_batch.rs:395-425. */
void orc_merge_head(int hd, int n_parts, const float* parts, size_t part_stride,
                    const float* sink, float* out);

typedef struct OrcDesc {
    int32_t n_head, n_kv, hd;
    int32_t n_seq;            /* sequences */
    int32_t q_tokens;         /* query tokens per sequence: the last q_tokens positions */
    const int32_t* seq_kv_len;    /* host [n_seq] keys per sequence */
    const int64_t* seq_kv_off;    /* host [n_seq] first cache row of each sequence */
    int64_t kv_row_stride;    /* f16 elements between consecutive cache rows */
    int32_t window;           /* 0 = all keys */
    int32_t ring_cap;         /* 0 = linear rows; else key position j lives in row j % ring_cap */
    float scale;              /* applied to q before the dot products */
} OrcDesc;

/* Attention of every query token: token t of sequence s sits at position
 * len_s - q_tokens + t and sees keys [lo, pos] (lo = pos+1-window when a
 * window is set).  Keys go through orc_chunk in 256-position chunks aligned
 * to absolute positions, the chunk partials are merged in order with the
 * sink.  q, out: [n_seq][q_tokens][n_head][hd] f32.  Tokens outside
 * [t_begin, t_end) are skipped (out untouched).  threads <= 0: all.
 * Returns 0, or -1 on a bad descriptor. */
int orc_attn(const OrcDesc* d, const float* q, const uint16_t* k, const uint16_t* v,
             const float* sinks, float* out, int t_begin, int t_end, int threads);

/* Prefill flavour: q and out are f16 ([n_seq][q_tokens][n_head][hd]), the
 * sums are f32 as in orc_attn, the output rounded to f16 (nearest even). */
int orc_attn_f16(const OrcDesc* d, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                 const float* sinks, uint16_t* out, int t_begin, int t_end, int threads);

/* Partials only: the chunks of keys [k_begin, k_end) of one decode token
 * (sequence s, token t) as (max, sum, O[hd]) per head, n_head*(hd+2) floats
 * per 256-position chunk slot, one slot per chunk from k_begin/256 on. This
 * is the CPU tier's output in src/moe.rs:1686-1712. Returns slots written. */
int orc_partials(const OrcDesc* d, const float* q, const uint16_t* k, const uint16_t* v,
                 int s, int t, int k_begin, int k_end, float* parts, int threads);

/* ---- the step before attention (oracle/qkv_oracle.c) ------------------ */

/* Rotary table: (cos, sin) pairs, rot/2 pairs per row.  table_split == 0:
 * row = position (ROPE_KV_T's table, src/oss_batch.rs:151-152, built by
 * src/oss.rs:1320-1349).  table_split = n > 0: rows < n hold positions 256 i,
 * rows n + p the positions p < 256, and a position's angle is composed from
 * rows pos/256 and n + pos%256 by angle addition (qk_dec,
 * src/moe_kernels.rs:350-355; table src/moe.rs:484-519). */
typedef struct OrcRope {
    int32_t rot;          /* rotated dims: the first rot of each head (even, <= hd) */
    int32_t neox;         /* 1: pairs (j, j + rot/2); 0: pairs (2j, 2j + 1) */
    int32_t table_split;  /* see above */
    const float* table;
} OrcRope;

/* What follows the q, k, v projections, per token (token t of sequence s at
 * position len_s - q_tokens + t): per-head RMS norm of q and k heads when
 * q_norm / k_norm are given (x * inv * w, inv = 1/sqrt(sum x^2 / hd + eps)),
 * rope on q and k, q written back, k and v rounded to f16 (nearest even)
 * into cache row seq_kv_off[s] + (ring_cap ? pos % ring_cap : pos).
 * q: [n_seq][q_tokens][n_head][hd], k, v: [n_seq][q_tokens][n_kv][hd] f32.
 * qk_dec (src/moe_kernels.rs:304-378), ROPE_KV_T (src/oss_batch.rs:113-170).
 * Returns 0, or -1 on a bad descriptor. */
int orc_qk_norm_rope_cache(const OrcDesc* d, const OrcRope* r, float* q, const float* k, const float* v,
                           const float* q_norm, const float* k_norm, float eps,
                           uint16_t* k_cache, uint16_t* v_cache);

#ifdef __cplusplus
}
#endif
#endif
