/* pelica_attn — MI355X (gfx950) attention for Pelica's decode and prefill
 * passes, behind a plain C ABI.
 *
 * All tensor pointers are DEVICE pointers owned by the caller; every call is
 * asynchronous on `stream` (a hipStream_t passed as void*, NULL = the null
 * stream).  No call allocates device memory except through the caller's
 * workspace.  No C++ exception crosses this boundary: every entry point
 * returns a status (0 ok, negative error) and the message of the calling
 * thread's last error is available from pelica_attn_last_error().
 *
 * Layouts (f16 = IEEE binary16 stored as uint16_t):
 *   q, out   token i = s * q_tokens + t holds its n_head * hd values (head
 *            h at h * hd) starting at element i * q_token_stride (q) or
 *            i * out_token_stride (out); stride 0 = n_head * hd, i.e.
 *            [n_seq][q_tokens][n_head][hd].  A nonzero stride lets the
 *            queries stay in place in the engine's fused [q | k | v] rows
 *            and the output go straight into a wider activation row, as
 *            the reference's kernels read and write them (q stride arg 9,
 *            out stride arg 10: src/oss_batch.rs:172-176,267-270,
 *            src/oss_prefill.rs:400-402, set at src/oss.rs:680,690,693,739).
 *   k, v     cache rows of n_kv*hd values, row r at k + r*kv_row_stride;
 *            key position j of sequence s lives in row
 *            seq_kv_offset[s] + (ring_cap ? j % ring_cap : j)
 *   sinks    [n_head] f32 logits (natural-log units) or NULL
 *   partials [slot][n_head][hd + 2] f32 (max, sum, hd sums of v) — the
 *            reference's merge_dec / cpu_attn partial format.
 *
 * Token t of sequence s is the query at position kv_len_s - q_tokens + t and
 * sees keys [lo, pos] with lo = max(0, pos + 1 - window) when a window is
 * set (causal among the pass's own tokens: drafts and prompt rows).
 *
 * The reference (HumandubleOfficial/Pelica) has no single attention function:
 * each entry point below replaces a set of WGSL dispatches recorded by its
 * engines, cited per function.
 */
#ifndef PELICA_ATTN_H
#define PELICA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PELICA_ATTN_VERSION 2

/* status codes */
#define PELICA_ATTN_OK 0
#define PELICA_ATTN_EINVAL (-1)      /* bad descriptor or argument */
#define PELICA_ATTN_EUNSUPPORTED (-2) /* valid but not implemented (e.g. hd) */
#define PELICA_ATTN_EHIP (-3)        /* a HIP runtime call failed */
#define PELICA_ATTN_EWORKSPACE (-4)  /* workspace missing or too small */

/* Shape and addressing of one attention call.  Replaces the 16-word u32
 * argument blocks of the reference's attention kernels
 * (src/moe_kernels.rs:39-43 arg(), src/oss.rs:760-778 params; fields of
 * src/cpu_attn.rs:13-26 Shape: hd, n_kv, hpk = n_head / n_kv). */
typedef struct PelicaAttnDesc {
    int32_t n_head;    /* query heads */
    int32_t n_kv;      /* kv heads; n_head % n_kv == 0 (GQA group n_head/n_kv) */
    int32_t hd;        /* dims per head: 64 or 128 */
    int32_t n_seq;     /* sequences in the batch (>= 1) */
    int32_t q_tokens;  /* query tokens per sequence: 1 decode, <= 8 drafts, T prompt */
    int32_t kv_len;    /* keys per sequence; with seq_kv_len set, an upper bound
                          (larger seq_kv_len entries are clipped to it) */
    const int32_t* seq_kv_len;    /* device [n_seq] keys per sequence, or NULL */
    const int64_t* seq_kv_offset; /* device [n_seq] first cache row, or NULL:
                                     sequence s then starts at row s * (ring_cap ? ring_cap : kv_len) */
    int64_t kv_row_stride; /* f16 values between cache rows; 0 = n_kv * hd */
    int32_t window;    /* sliding window in keys, 0 = all (src/oss_batch.rs:175) */
    int32_t ring_cap;  /* 0 = linear cache; else rows of a ring of ring_cap positions
                          (src/oss_batch.rs:205, src/oss.rs:570-572) */
    float scale;       /* logit scale; 0 = 1/sqrt(hd) (src/moe.rs:1263) */
    uint32_t flags;    /* 0, or PELICA_ATTN_FLAG_SPLIT_ONLY (pelica_attn_decode only) */
    int64_t q_token_stride;   /* elements between consecutive query tokens; 0 = n_head * hd.
                                 A multiple of 4 (f32 queries) or 8 (f16), >= n_head * hd */
    int64_t out_token_stride; /* elements between consecutive output tokens; 0 = n_head * hd.
                                 A multiple of 4 (f32 output) or 8 (f16), >= n_head * hd */
} PelicaAttnDesc;

/* Measurement flag (no counterpart in the reference): pelica_attn_decode
 * skips the combine of the key splits, leaving the split partials in the
 * workspace (`out` holds the result only when the call has one split), so a
 * profiler or a graph of such calls times the split kernel alone.  Rejected
 * by every other entry point. */
#define PELICA_ATTN_FLAG_SPLIT_ONLY 1u

/* PELICA_ATTN_VERSION of the loaded library. */
int pelica_attn_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char* pelica_attn_last_error(void);

/* Measurement and test switch (no counterpart in the reference): the
 * planner's PELICA_ATTN_* tuning variables are read from the environment
 * once, at the first call that plans a pass; this re-reads them.  Plans and
 * workspace sizes may change with it: size workspaces again afterwards.
 * Calls planned concurrently with it use either the old or the new values. */
int pelica_attn_reload_tuning(void);

/* Bytes of device workspace pelica_attn_decode needs for this descriptor
 * (split-K partials).  0 on an invalid descriptor (see last_error) or when
 * the call needs none.  Its contents need no initialisation; calls that
 * share one workspace must be ordered on one stream.
 * Replaces the partials buffer `part` (src/moe.rs:949-952) and the split
 * partials of attn_s (src/oss.rs:573-576). */
size_t pelica_attn_workspace_bytes(const PelicaAttnDesc* desc);

/* Zero-fill a workspace on `stream` with a fill kernel (safe to record in a
 * HIP graph).  Decode does not require it; it is there for callers that
 * want deterministic workspace contents.  No counterpart in the reference,
 * whose wgpu buffers start zeroed at creation (src/moe.rs:949-952). */
int pelica_attn_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/* Decode attention: f32 queries over the f16 cache, f32 output, split-K
 * flash-decode plus an in-order combine with the sinks.
 * Replaces: attn_dec / attn_dec_fast + merge_dec (src/moe_kernels.rs:482-808,
 * dispatched at src/moe.rs:1343,1364), ATTN_T (src/oss_batch.rs:172-251,
 * src/oss.rs:675-683), attn_s + ATTN_M (src/oss_batch.rs:253-425,
 * src/oss.rs:685-693) and the draft-verify pass of those (T <= 8). */
int pelica_attn_decode(const PelicaAttnDesc* desc, const float* q, const uint16_t* k,
                       const uint16_t* v, const float* sinks, float* out,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Decode without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The same pass and result
 * as pelica_attn_decode, with its split partials in a static device array
 * of PELICA_ATTN_NOALLOC_SCRATCH_BYTES that each GPU the library runs on
 * holds until the process ends; a pass that needs more (see
 * pelica_attn_workspace_bytes) is rejected with PELICA_ATTN_EWORKSPACE.
 * The call allocates nothing.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race
 * and must be ordered by the caller, e.g. on one stream.  The array's
 * contents need no clearing between calls (each pass writes every scratch
 * value it reads).  The first call on a device looks up its copy of the
 * array with that device current; `stream` must belong to the current
 * device. */
#define PELICA_ATTN_NOALLOC_SCRATCH_BYTES (16u << 20)
int pelica_attn_decode_noalloc(const PelicaAttnDesc* desc, const float* q, const uint16_t* k,
                               const uint16_t* v, const float* sinks, float* out, void* stream);

/* Decode partials: the same pass as pelica_attn_decode, but instead of the
 * output it writes the (max, sum, unnormalised O) of the keys this cache
 * holds, one slot per (sequence, token, head) in merge_dec's format:
 *   parts[((s*q_tokens + t)*n_head + h)*(hd+2)] = {M, L, O[0..hd)},
 * M the natural-log max of the scaled scores (-3e38 when no key is
 * visible), L = sum e^(s-M), O = sum e^(s-M) v.  No sinks: they join in the
 * final pelica_attn_partials_merge together with the CPU tier's slots.
 * Workspace as for pelica_attn_decode.  Replaces dec_res, attn_dec over the
 * VRAM rows into the partial slots `part` (src/moe.rs:1600-1606,
 * src/moe_kernels.rs:482-583), that src/moe.rs:1713-1729 completes with
 * the rows past VRAM. */
int pelica_attn_decode_partials(const PelicaAttnDesc* desc, const float* q, const uint16_t* k,
                                const uint16_t* v, float* parts, void* workspace,
                                size_t workspace_bytes, void* stream);

/* Decode partials over one range of key positions [key_begin, key_end)
 * whose cache rows start at k_rows / v_rows (row 0 = position key_begin),
 * e.g. the rows past `res` that the reference keeps in host memory (its
 * "far" buffers).  Same slots and workspace as pelica_attn_decode_partials
 * (rows that see no key of the range get M = -3e38, L = 0, O = 0); one
 * sequence (n_seq 1, no seq_kv_len), linear cache (ring_cap 0);
 * 0 <= key_begin < key_end <= kv_len.  The reference's attn_s reads its
 * keys below res from VRAM and the rest from the far buffers in one
 * dispatch (src/oss_batch.rs:253-393, args 3 and 10; src/oss.rs:685-693);
 * here that pass is two of these calls, [0, res) over the VRAM rows and
 * [res, kv_len) over the far rows, whose slots pelica_attn_partials_merge_batch
 * combines with the sinks (ATTN_M, src/oss_batch.rs:395-425). */
int pelica_attn_decode_partials_range(const PelicaAttnDesc* desc, const float* q, const uint16_t* k_rows,
                                      const uint16_t* v_rows, int32_t key_begin, int32_t key_end,
                                      float* parts, void* workspace, size_t workspace_bytes,
                                      void* stream);

/* MLA (latent) attention: one kv head whose keys and values are the same
 * latent cache rows, hd = 512 f16 per position (row stride kv_row_stride,
 * 0 = 512); n_kv must be 1; q: the absorbed f32 queries
 * [n_seq][q_tokens][n_head][512], out f32 alike; token t sees positions
 * <= len - q_tokens + t (causal, no window, no sinks); scale as given (the
 * engine passes 1/sqrt(qk_nope)).  Workspace from
 * pelica_attn_mla_workspace_bytes.  Replaces mla (src/gpu.rs:262-307,
 * src/forward.rs:936-960), whose latent cache is f32; the f16 rows here are
 * the same switch as gpt-oss's. */
size_t pelica_attn_mla_workspace_bytes(const PelicaAttnDesc* desc);
int pelica_attn_mla(const PelicaAttnDesc* desc, const float* q, const uint16_t* latent, float* out,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Prefill (prompt) attention: f16 queries, f16 cache, f16 output, f32
 * accumulation and softmax, causal with optional window and sinks.
 * Replaces: attn_p (src/oss_prefill.rs:391-526, src/oss.rs:734-741) and
 * attn_pre + attn_fold (src/moe_kernels.rs:810-990, src/moe.rs:1345-1362). */
int pelica_attn_prefill(const PelicaAttnDesc* desc, const uint16_t* q, const uint16_t* k,
                        const uint16_t* v, const float* sinks, uint16_t* out, void* stream);

/* The same prompt attention with f32 queries and f32 output, the layout
 * the reference's attn_p reads and writes (q f32 rows at stride qkv_rows,
 * xo f32 at stride attw: src/oss_prefill.rs:391-526, src/oss.rs:734-741).
 * The queries are rounded to f16 for the QK^T products (as the f16 cache
 * rows are); softmax and accumulation stay f32. */
int pelica_attn_prefill_f32(const PelicaAttnDesc* desc, const float* q, const uint16_t* k,
                            const uint16_t* v, const float* sinks, float* out, void* stream);

/* Prompt attention over one round of keys: the cache rows of key positions
 * [key_begin, key_end) (k_rows / v_rows row 0 = position key_begin, e.g. a
 * staging copy of rows that live past HBM) folded into a running state per
 * (token, head), state[(t*n_head + h)*(hd+2)] = {M natural-log, L, O[hd]}
 * (unnormalised), f32.  first = 1 starts the state empty (its contents are
 * not read).  Rounds must come in key order; after the round that holds key
 * position len-1 the state is complete.  out (optional, f16
 * [q_tokens][n_head][hd]) receives the output so far, with the sinks, 0 for
 * rows that have seen no key.  One sequence, linear cache; causal and window
 * masks as pelica_attn_prefill.  Replaces attn_pre + attn_fold over
 * 16K-key rounds of VRAM and staged rows (src/moe_kernels.rs:810-990,
 * dispatched src/moe.rs:1609-1627). */
int pelica_attn_prefill_round(const PelicaAttnDesc* desc, const uint16_t* q, const uint16_t* k_rows,
                              const uint16_t* v_rows, int32_t key_begin, int32_t key_end,
                              const float* sinks, float* state, int32_t first, uint16_t* out,
                              void* stream);

/* prefill_round with f32 queries and f32 out (see pelica_attn_prefill_f32). */
int pelica_attn_prefill_round_f32(const PelicaAttnDesc* desc, const float* q, const uint16_t* k_rows,
                                  const uint16_t* v_rows, int32_t key_begin, int32_t key_end,
                                  const float* sinks, float* state, int32_t first, float* out,
                                  void* stream);

/* Combine n_parts partial slots of one decode token (parts[(c*n_head+h)*(hd+2)],
 * natural-log max) in slot order, with optional sinks, into out[n_head][hd].
 * Slots whose max is -3e38 (or -inf) carry no weight, as the reference's
 * empty slots do.  hd even, <= 1024; parts and out 8-byte aligned.
 * Replaces merge_dec (src/moe_kernels.rs:585-617) and ATTN_M's combine
 * (src/oss_batch.rs:395-425); it is how partials from the CPU tier
 * (cpu_attn::chunk, src/moe.rs:1686-1729) join the GPU's.  Same as
 * pelica_attn_partials_merge_batch with n_tokens = 1. */
int pelica_attn_partials_merge(int32_t n_head, int32_t hd, int32_t n_parts,
                               const float* parts, const float* sinks, float* out,
                               void* stream);

/* The same merge for n_tokens query tokens at once (e.g. n_seq * q_tokens
 * rows of a draft-verify pass): slot c of token t, head h at
 * parts[((c*n_tokens + t)*n_head + h)*(hd+2)], output out[t][n_head][hd]
 * (so the slots that pelica_attn_decode_partials writes for a whole pass are
 * one slot c here).  Every thread loads its slots in one round trip and
 * computes their weights itself (no staging barrier).
 * Replaces ATTN_M over its (n_head, TMAX) grid (src/oss_batch.rs:395-425)
 * and merge_dec_fast (src/moe_kernels.rs:750-808). */
int pelica_attn_partials_merge_batch(int32_t n_tokens, int32_t n_head, int32_t hd, int32_t n_parts,
                                     const float* parts, const float* sinks, float* out,
                                     void* stream);

/* ---- the step before attention ----------------------------------------- */

/* Rotary embedding table: (cos, sin) float pairs, rot/2 pairs per row.
 * table_split == 0: row = position (the gpt-oss table, src/oss.rs:1320-1349,
 * read at src/oss_batch.rs:151-152).  table_split = n > 0: the two-level
 * table of src/moe.rs:484-519 — rows < n hold positions 256 i, rows n + p
 * the positions p < 256 — composed by angle addition
 * (src/moe_kernels.rs:350-355). */
typedef struct PelicaRope {
    int32_t rot;          /* rotated dims at the start of each head: even, <= hd; 0 = no rope */
    int32_t neox;         /* 1: pairs (j, j + rot/2) (NeoX, gpt-oss); 0: pairs (2j, 2j + 1) */
    int32_t table_split;  /* 0, or the number of 256-position rows (see above) */
    int32_t table_rows;   /* rows in table (positions are checked against it) */
    const float* table;   /* device [table_rows][rot/2][2] */
} PelicaRope;

/* What follows the q, k, v projections of the pass's tokens, in one launch:
 * per-head RMS norm of q and k heads (x * inv * w, inv = 1/sqrt(mean x^2 +
 * eps)) when q_norm / k_norm are given, rope on q and k, q written back in
 * place, the k and v rows rounded to f16 into the cache.  Token t of
 * sequence s sits at position len_s - q_tokens + t and its row is
 * seq_kv_offset[s] + (ring_cap ? pos % ring_cap : pos) (as for attention).
 * q: [n_seq*q_tokens tokens][n_head][hd], k, v: [tokens][n_kv][hd] f32; token
 * i's heads start at i * token_stride floats (0: dense per tensor; the
 * engine's fused [q | k | v] rows use (n_head + 2 n_kv) hd).  hd: 64, 128
 * or 256.  Replaces qk_dec (src/moe_kernels.rs:304-378, src/moe.rs:1322-1340)
 * and ROPE_KV_T (src/oss_batch.rs:113-170), writing f16 rows where gpt-oss
 * kept f32 ones (src/oss.rs:615-616). */
int pelica_attn_qkv_rope_cache(const PelicaAttnDesc* desc, const PelicaRope* rope, float* q,
                               const float* k, const float* v, int64_t token_stride,
                               const float* q_norm, const float* k_norm, float eps,
                               uint16_t* k_cache, uint16_t* v_cache, void* stream);

/* ---- per-kernel GPU timing ------------------------------------------- */

/* kernel ids of PelicaAttnProfRecord */
#define PELICA_ATTN_PROF_DECODE_SPLIT 1
#define PELICA_ATTN_PROF_DECODE_COMBINE 2
#define PELICA_ATTN_PROF_PREFILL 3
#define PELICA_ATTN_PROF_MERGE 4
#define PELICA_ATTN_PROF_QKV 5

typedef struct PelicaAttnProfRecord {
    int32_t kernel; /* PELICA_ATTN_PROF_* */
    float ms;       /* GPU time between the events bracketing the launch */
} PelicaAttnProfRecord;

/* Turn per-kernel timing on (1) or off (0); either way pending records are
 * dropped.  While on, each kernel launch is bracketed by HIP events on its
 * stream (launches on a capturing stream are not timed).  Replaces the
 * reference's PELICA_PROF timestamp queries (src/moe.rs:1761-1833,
 * src/oss.rs:1164-1242). */
int pelica_attn_prof_enable(int on);

/* Wait for the recorded launches, copy up to max_records of them (in launch
 * order) to out and drop all records.  Returns the number copied, or a
 * negative status. */
int pelica_attn_prof_read(PelicaAttnProfRecord* out, int max_records);

#ifdef __cplusplus
}
#endif
#endif
