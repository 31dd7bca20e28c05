/*
 * mrml_oracle.h -- CPU oracle for the MRML decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the GPU backend is
 * compared against; it is never part of the product path.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * It is a plain-C restatement of the reference's CPU kernels
 * (crates/mrml-tensor/src/quant.rs, ops.rs, parallel.rs, kv_cache.rs,
 * model.rs of mitchellrenouf/QT_llama.cpp); each function's comment cites
 * the reference lines it follows.  Compiled with -ffp-contract=off and no
 * fast-math so every float operation rounds exactly where the Rust source
 * rounds (Rust never contracts a*b+c into an FMA).
 *
 * Parity pins (what checks each function beyond its own formula) are listed
 * per function; functions marked "build-defined" have no counterpart in the
 * reference and are pinned by closed forms and brute force only.
 */
#ifndef MRML_ORACLE_H
#define MRML_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 / bf16 scalar conversions (quant.rs:47-116) ------------------ */
float    orc_f16_to_f32(uint16_t h);          /* quant.rs:47-77, exact        */
uint16_t orc_f32_to_f16(float f);             /* quant.rs:81-104, truncating  */
/* Round-to-nearest-even f32->f16 (IEEE 754).  Used for the f16 KV cache of
 * the build-defined decode step, matching the reference GPU path's cvt.rn
 * (cuda_ptx/kernels.rs:1321).  Overflow -> Inf, subnormals kept. */
uint16_t orc_f32_to_f16_rne(float f);

/* ---- block codecs ------------------------------------------------------ */
/* quant.rs:193-228.  n % 32 == 0; dst holds n/32 * 34 bytes. */
void orc_quantize_q8_0(const float *src, uint8_t *dst, size_t n);
/* quant.rs:166-190 */
void orc_dequantize_q8_0(const uint8_t *src, float *dst, size_t n);
/* quant.rs:135-163 */
void orc_dequantize_q4_0(const uint8_t *src, float *dst, size_t n);
/* quant.rs:372-389 */
void orc_quantize_q4_0(const float *src, uint8_t *dst, size_t n);

/* ---- block dot products ----------------------------------------------- */
/* isa: 0 = scalar (quant.rs:335-369), 1 = AVX2 (quant.rs:272-332),
 *      2 = AVX-VNNI (quant.rs:443-479), -1 = the reference's own dispatch
 *      (quant.rs:252-268: VNNI if CPUID.(7,1):EAX[4], else AVX2, else scalar).
 * Returns NaN if the requested ISA is not available on this host. */
float orc_vec_dot_q4_0_q8_0(const uint8_t *w, const uint8_t *a, size_t n, int isa);
/* quant.rs:484-577.  The AVX2 variant folds in a different order
 * (8 lane accumulators, quant.rs:534-561) and may differ in the last bits. */
float orc_vec_dot_q8_0_q8_0(const uint8_t *x, const uint8_t *y, size_t n, int isa);
/* Per-block integer accumulators of the Q4_0 x Q8_0 dot (the exact int32
 * isum_b of quant.rs:352-363), nb = n/32 values. */
void orc_block_isums_q4_0_q8_0(const uint8_t *w, const uint8_t *a, size_t n, int32_t *isum);
/* Same for Q8_0 x Q8_0 (quant.rs:570-573). */
void orc_block_isums_q8_0_q8_0(const uint8_t *x, const uint8_t *y, size_t n, int32_t *isum);

/* Host ISA the dispatcher picks: 2 VNNI, 1 AVX2, 0 scalar. */
int orc_host_isa(void);

/* ---- matvec (ops.rs:162-260 over parallel.rs:73-116) ------------------- */
/* y[r] = vec_dot_q4_0_q8_0(W[r], x_q8).  threads <= 1 runs serially;
 * otherwise rows are split like parallel::for_each_range(len, 64). */
void orc_mat_vec_mul_q4_0_q8_0(const uint8_t *w, const uint8_t *x_q8, float *y,
                               size_t rows, size_t cols, int isa, int threads);
/* ops.rs:162-180: quantizes x itself first. */
void orc_mat_vec_mul_q4_0(const uint8_t *w, const float *x, float *y,
                          size_t rows, size_t cols, int isa, int threads);
/* model.rs:2842-2861 vocabulary loop: y[r] = vec_dot_q8_0_q8_0(W[r], x_q8),
 * then 30*tanh(y/30) if softcap != 0 (model.rs:2853). */
void orc_mat_vec_mul_q8_0_q8_0(const uint8_t *w, const uint8_t *x_q8, float *y,
                               size_t rows, size_t cols, int softcap, int isa, int threads);

/* ---- Q4_K (build-defined; the reference has no Q4_K dot) --------------- */
/* GGUF Q4_K super-block (144 B / 256 weights) dequantised by the public GGUF
 * rule.  The reference's dequantize_q4_k_to_f32 (quant.rs:598-638) uses a
 * different, non-GGUF scale/nibble order; this build follows GGUF. */
void orc_dequantize_q4_k(const uint8_t *src, float *dst, size_t n);
/* Unpack the 6-bit (scale, min) pair of sub-block j (0..7). */
void orc_q4_k_scale_min(const uint8_t *scales12, int j, uint8_t *sc, uint8_t *m);
/* Dot of one Q4_K row with a Q8_0 activation vector.  Per sub-block j with
 * the aligned Q8_0 block (d_a, a):
 *   isum_j = sum q*a, bsum_j = sum a                 (exact int32)
 *   t_j = (float)isum_j*((d*(float)sc_j)*d_a) - (float)bsum_j*((dmin*(float)m_j)*d_a)
 *   y   = sequential fold of t_j over super-blocks, then j, no FMA. */
float orc_vec_dot_q4_k_q8_0(const uint8_t *w, const uint8_t *a, size_t n);
void orc_mat_vec_mul_q4_k_q8_0(const uint8_t *w, const uint8_t *x_q8, float *y,
                               size_t rows, size_t cols, int threads);

/* ---- greedy selection (model.rs:2833-2907; GPU tie rule kernels.rs:1144) */
/* Index of the maximum; NaN never wins; ties go to the lowest index. */
int64_t orc_argmax_f32(const float *x, size_t n);

/* Vocabulary scoring and the next-token pick of step_generation
 * (model.rs:2842-2907):
 *   candidates: tokens with valid[id] != 0 (valid nullable: all), minus ids
 *     1, 2, 105, 106 while generated_count < 4;
 *   scoring 0 (CPU path, model.rs:2852-2856): logits are raw dot products;
 *     score = 30 * tanhf(logit / 30), then -3.5 when id is one of the
 *     n_recent ids of recent (once, however often it occurs);
 *   scoring 1 (device path, kernels.rs:1110-1123 after the softcapping Q8
 *     GEMV): score = logit, -1.8 for each occurrence of id in recent;
 *   NaN scores are not candidates;
 *   the k best by score, descending; equal scores by ascending id (the
 *     reference's unstable sorts leave that order open; this is the GPU
 *     kernels' rule, kernels.rs:1144-1145);
 *   temperature <= 0: the first; else p_i = expf((s_i - s_0) / max(t, 0.1))
 *     summed in order, rng = (f32)((pos * 6364136223846793005 + 1) >> 33) /
 *     (f32)UINT32_MAX, and the first i with rng <= (acc += p_i / sum);
 *   no candidate: token 506 (the reference's fallback).
 * Writes the n_out = min(k, #candidates) best (score, id) to out_scores /
 * out_ids (each nullable) and returns the token. */
int32_t orc_vocab_select(const float *logits, size_t vocab, const uint8_t *valid, const int32_t *recent,
                         size_t n_recent, size_t generated_count, int scoring, float temperature, uint64_t pos,
                         size_t k, float *out_scores, int32_t *out_ids, size_t *n_out);

/* ---- elementwise / normalisation (ops.rs) ------------------------------ */
void  orc_rms_norm(const float *x, const float *w, float eps, float *out, size_t dim); /* ops.rs:24-49 */
void  orc_rope_1d(float *v, size_t pos, size_t head_dim, float base, float scale);   /* ops.rs:82-97 */
void  orc_rope_1d_batched(float *v, size_t pos, size_t n_heads, size_t head_dim,
                          float base, float scale);                                    /* ops.rs:185-208 */
float orc_gelu_approx(float x);                                                        /* ops.rs:101-104 */
void  orc_geglu(const float *gate, const float *up, float *out, size_t n);             /* ops.rs:107-114 */
float orc_silu(float x);                                                               /* ops.rs:118-120 */
void  orc_swiglu(const float *gate, const float *up, float *out, size_t n);            /* ops.rs:123-130 */
void  orc_softmax(float *x, size_t n);                                                 /* ops.rs:133-158 */

/* ---- decode attention over an f16 KV cache (build-defined composition of
 * model.rs:1457-1590 with an F32-format dot and an f16 cache) ----------- */
/* q: n_heads*head_dim; k_cache/v_cache: [pos][n_kv_heads][head_dim] f16 bits.
 * Positions 0..n_past inclusive are attended.  scores_t = (q.k_t)*scale,
 * softmax, out = sum_t p_t*v_t in position order. */
void orc_attention_f16(const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                       float *out, size_t n_past, size_t n_heads, size_t n_kv_heads,
                       size_t head_dim, float scale);

/* ---- KV cache formats (kv_cache.rs:8-125; KvCacheFormat::cuda_code 0 f16,
 * 1 Q8_0, 2 Q4_0) ---------------------------------------------------------- */
/* Bytes of n cached values in format fmt (n % 32 == 0 for 1 and 2). */
size_t orc_kv_row_bytes(size_t n, int fmt);
/* KvCacheRow::from_f32: f16 (round to nearest even), quantize_f32_to_q8_0 or
 * quantize_f32_to_q4_0 of n values. */
void   orc_kv_store(const float *x, uint8_t *dst, size_t n, int fmt);
/* KvCacheRow::dot_head: q . k of one head's cached keys; q8 =
 * quantize_f32_to_q8_0(q) (read for formats 1 and 2 only). */
float  orc_kv_dot_head(const uint8_t *row, const float *q, const uint8_t *q8, size_t head_dim, int fmt);
/* KvCacheRow::add_head_scaled: out += p * v of one head's cached values. */
void   orc_kv_add_head_scaled(const uint8_t *row, float *out, size_t head_dim, float p, int fmt);
/* Attention over caches of those formats (model.rs:1526-1547): positions
 * 0..n_past of [pos][n_kv_heads][head_dim] rows in the formats' bytes. */
void   orc_attention_kv(const float *q, const uint8_t *k_cache, const uint8_t *v_cache, float *out, size_t n_past,
                        size_t n_heads, size_t n_kv_heads, size_t head_dim, float scale, int k_fmt, int v_fmt);

/* ---- Gemma-2-2B-shape decode step (build-defined composition) ---------- */
typedef struct orc_gemma2 {
    int32_t n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim, vocab, ctx;
    float   rope_base, eps, attn_scale;
    int32_t tie_q8;          /* 0: tied table is Q4_0, 1: Q8_0 */
    int32_t softcap;         /* apply 30*tanh(x/30) to the logits */
    int32_t sliding_window;  /* > 0: windowed layers attend the last sliding_window positions */
    int32_t swa_period;      /* layer l is windowed unless l % swa_period == swa_period - 1 */
    const uint8_t *tok_embd; /* vocab rows of dim, GGUF bytes */
    const float   *output_norm;
    /* per-layer arrays of n_layers pointers */
    const uint8_t *const *wq, *const *wk, *const *wv, *const *wo;
    const uint8_t *const *wgate, *const *wup, *const *wdown;
    const float *const *attn_norm, *const *post_attn_norm;
    const float *const *ffn_norm, *const *post_ffw_norm;
} orc_gemma2;

/* One token through the model at position pos.  k_cache/v_cache are
 * per-layer [ctx][n_kv_heads][head_dim] f16 arrays, laid end to end
 * (layer-major).  Writes logits[vocab] (may be NULL) and returns the greedy
 * token.  threads parallelises the matvecs only (results do not depend on it). */
int64_t orc_gemma2_step(const orc_gemma2 *m, int64_t token, int64_t pos,
                        uint16_t *k_cache, uint16_t *v_cache, float *logits, int threads);

#ifdef __cplusplus
}
#endif
#endif
