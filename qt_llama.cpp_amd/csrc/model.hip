// model.hip -- C ABI of the decode-step ops and the Gemma-2-shape token step.
//
// The reference composes a token step in model.rs (forward_token,
// model.rs:1185-2260; greedy selection model.rs:2833-2907) from CudaDevice
// calls.  mrml_hip_gemma2_step enqueues the same composition on the
// context's stream, reading the token and position from device memory and
// advancing them in its last kernel, so one captured graph of a step replays
// for every prompt and generated token without a host round trip.
//
// Per layer (9 launches):
//   qkv      = [Wq|Wk|Wv] * pack(xn)                      gemv_q4_0_qkv
//   RoPE(q, k); k, v -> f16 cache row pos                  rope_kv_f16
//   attn     = softmax(scale * q K^T) V  -> Q8_0 pack      attn partial + combine
//   o        = Wo * pack(attn)                             gemv_q4_0
//   h += rms_norm(o, post_attn); xn = rms_norm(h, ffn)    residual_rms_norm -> pack
//   act      = gelu(Wg xn) * (Wu xn)     -> Q8_0 pack      gemv_q4_0_geglu (emit)
//   f        = Wd * pack(act)                              gemv_q4_0 (long-row kernel)
//   h += rms_norm(f, post_ffw); xn = rms_norm(h, next)    residual_rms_norm -> pack
// then the tied LM head over pack(rms_norm(h, output_norm)) and the pick:
// argmax, or with a sampler the reference's scoring and draw.

#include <algorithm>
#include <cmath>
#include <new>
#include <vector>

#include "device.h"
#include "internal.h"

// scores of the attention rows of one batched launch held at once
static constexpr size_t kPrefillScoreBytes = 64u << 20;

struct mrml_hip_gemma2 {
    mrml_hip_gemma2_config cfg{};
    const void *tok_embd = nullptr;
    const float *output_norm = nullptr;
    std::vector<mrml_hip_gemma2_layer> layers;
    void *arena = nullptr;  // activations, packs, partials (one allocation)
    float *h = nullptr, *qkv = nullptr, *o = nullptr, *f = nullptr, *logits = nullptr;
    float *h2 = nullptr;  // the residual's other buffer when the residual runs inside the matvecs
    float *act = nullptr;  // f32 GeGLU output of the unfused path (never the context workspace, which
                           // may be reallocated under a captured graph)
    uint8_t *xpack = nullptr, *attn_pack = nullptr, *act_pack = nullptr;
    void *attn_part = nullptr, *argmax_scratch = nullptr;
    void *recent_ring = nullptr;    // {position, token} of the last 32 positions processed
    void *select_scratch = nullptr;  // partition keys of the sampler's pick
    mrml_hip_sampler sampler{};      // top_k == 0: plain argmax
    float *rope_table = nullptr;  // [ctx_len][head_dim/2] (cos, sin) from the host libm
    float *rope_freqs = nullptr;  // [head_dim/2] powf(base, 2i/head_dim) from the host libm (positions >= ctx_len)
    // prefill chunk buffers, allocated on the first prefill call: per token
    // rows of h, xn, stacked q|k|v, attention output, o, stacked gate|up and f,
    // plus one GEMM pack (act is quantized into it as it is formed)
    void *pf_arena = nullptr;
    float *pf_h = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr,
          *pf_attn = nullptr, *pf_o = nullptr, *pf_gu = nullptr, *pf_f = nullptr;
    void *pf_gpack = nullptr, *pf_scores = nullptr;  // GEMM pack; attention scores of every row
};

using namespace mrml;

namespace {

constexpr int kSamplerTopKMax = 64;

int check_model_config(mrml_hip_ctx *ctx, const mrml_hip_gemma2_config &c)
{
    REQUIRE(ctx, c.n_layers > 0 && c.dim > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.ffn_dim > 0 &&
                     c.vocab > 0 && c.ctx_len > 0,
            "gemma2: every size must be positive");
    REQUIRE(ctx, c.head_dim == attn_head_dim(), "gemma2: head_dim %d unsupported (the attention kernel serves %d)",
            c.head_dim, attn_head_dim());
    REQUIRE(ctx, c.n_heads % c.n_kv_heads == 0 && c.n_heads / c.n_kv_heads <= 8,
            "gemma2: n_heads=%d must be a multiple of n_kv_heads=%d with a group of at most 8", c.n_heads,
            c.n_kv_heads);
    REQUIRE(ctx, norm_dim_ok(c.dim), "gemma2: dim=%d must be a multiple of 32 up to 12288", c.dim);
    REQUIRE(ctx, c.ffn_dim % 32 == 0, "gemma2: ffn_dim=%d must be a multiple of 32", c.ffn_dim);
    REQUIRE(ctx, c.tie_type == MRML_HIP_Q4_0 || c.tie_type == MRML_HIP_Q8_0,
            "gemma2: tie_type must be Q4_0 or Q8_0");
    REQUIRE(ctx, c.ctx_len <= attn_max_capacity(), "gemma2: ctx_len=%d above %d", c.ctx_len, attn_max_capacity());
    REQUIRE(ctx, c.numerics == MRML_HIP_NUMERICS_EXACT || c.numerics == MRML_HIP_NUMERICS_FAST,
            "gemma2: numerics=%d is neither EXACT (0) nor FAST (1)", c.numerics);
    REQUIRE(ctx, vocab_select_ok(c.vocab, kSamplerTopKMax), "gemma2: vocab=%d above the sampler's limit", c.vocab);
    REQUIRE(ctx, c.sliding_window >= 0 && c.swa_period >= 0, "gemma2: sliding_window=%d swa_period=%d",
            c.sliding_window, c.swa_period);
    return MRML_HIP_OK;
}

// Layer l's attention window limit for the attention launches: the sliding
// window on a windowed layer (model.rs:590, 1465-1467), else -1 (the cache).
int layer_window(const mrml_hip_gemma2_config &c, int l)
{
    return c.sliding_window > 0 && c.swa_period > 0 && l % c.swa_period != c.swa_period - 1 ? c.sliding_window : -1;
}

}  // namespace

extern "C" {

// ---- decode-step ops -------------------------------------------------------------

int mrml_hip_rms_norm(mrml_hip_ctx *ctx, const float *x, const float *w, float *out, void *pack, int32_t dim,
                      float eps)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, x && (out || pack), "rms_norm: x is null or no output requested");
    REQUIRE(ctx, norm_dim_ok(dim), "rms_norm: dim=%d must be a multiple of 32 up to 12288", dim);
    REQUIRE(ctx, ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                     ((uintptr_t)pack & 15) == 0,
            "rms_norm: pointers must be 16-byte aligned");
    return launch_rms_norm(ctx, x, w, eps, out, pack, dim);
}

int mrml_hip_rms_norm_batch(mrml_hip_ctx *ctx, const float *x, const float *w, float *out, int32_t dim, int32_t batch,
                            float eps)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, x && out, "rms_norm_batch: null pointer");
    REQUIRE(ctx, norm_dim_ok(dim), "rms_norm_batch: dim=%d must be a multiple of 32 up to 12288", dim);
    REQUIRE(ctx, batch > 0 && batch <= 65535, "rms_norm_batch: batch=%d (1..65535)", batch);
    REQUIRE(ctx, ((((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15) == 0),
            "rms_norm_batch: pointers must be 16-byte aligned");
    return launch_rms_norm(ctx, x, w, eps, out, nullptr, dim, batch);
}

int mrml_hip_residual_rms_norm(mrml_hip_ctx *ctx, const float *t, const float *w_post, float *h,
                               const float *w_next, float *xn, void *pack, int32_t dim, float eps)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, t && h, "residual_rms_norm: t and h are required");
    REQUIRE(ctx, norm_dim_ok(dim), "residual_rms_norm: dim=%d must be a multiple of 32 up to 12288", dim);
    REQUIRE(ctx, (((uintptr_t)t | (uintptr_t)w_post | (uintptr_t)h | (uintptr_t)w_next | (uintptr_t)xn |
                   (uintptr_t)pack) & 15) == 0,
            "residual_rms_norm: pointers must be 16-byte aligned");
    return launch_residual_rms_norm(ctx, t, w_post, h, h, w_next, eps, xn, pack, dim);
}

int mrml_hip_embedding(mrml_hip_ctx *ctx, const void *table, int32_t type, int32_t token, const int32_t *d_token,
                       float *out, int32_t dim, int32_t vocab, float scale)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, table && out, "embedding: null pointer");
    REQUIRE(ctx, type == MRML_HIP_Q4_0 || type == MRML_HIP_Q8_0, "embedding: type must be Q4_0 or Q8_0");
    REQUIRE(ctx, norm_dim_ok(dim) && vocab > 0, "embedding: dim=%d vocab=%d", dim, vocab);
    REQUIRE(ctx, d_token || (token >= 0 && token < vocab), "embedding: token %d outside [0, %d)", token, vocab);
    REQUIRE(ctx, ((uintptr_t)out & 15) == 0 && ((uintptr_t)table & 15) == 0,
            "embedding: pointers must be 16-byte aligned");
    return launch_embedding(ctx, table, type, d_token, token, scale, out, nullptr, 0.0f, nullptr, nullptr, dim, vocab);
}

int mrml_hip_rope_table(mrml_hip_ctx *ctx, float *d_table, int32_t n_pos, int32_t head_dim, float freq_base,
                        float freq_scale)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, d_table && n_pos > 0 && head_dim > 0 && head_dim % 2 == 0,
            "rope_table: n_pos=%d head_dim=%d", n_pos, head_dim);
    REQUIRE(ctx, ((uintptr_t)d_table & 7) == 0, "rope_table: table must be 8-byte aligned");
    return fill_rope_table(ctx, d_table, n_pos, head_dim, freq_base, freq_scale);
}

int mrml_hip_rope_kv_append_f16(mrml_hip_ctx *ctx, float *qkv, uint16_t *k_cache, uint16_t *v_cache, int32_t pos,
                                const int32_t *d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                float freq_base, float freq_scale, int32_t capacity, const float *d_table,
                                int32_t n_table)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, qkv && k_cache && v_cache, "rope_kv_append_f16: null pointer");
    REQUIRE(ctx, n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && head_dim <= 1024,
            "rope_kv_append_f16: n_heads=%d n_kv_heads=%d head_dim=%d", n_heads, n_kv_heads, head_dim);
    REQUIRE(ctx, capacity > 0 && (d_pos || pos >= 0), "rope_kv_append_f16: pos=%d capacity=%d", pos, capacity);
    REQUIRE(ctx, ((uintptr_t)d_table & 7) == 0 && n_table >= 0, "rope_kv_append_f16: table");
    return launch_rope_kv_f16(ctx, qkv, k_cache, v_cache, d_pos, pos, n_heads, n_kv_heads, head_dim, freq_base,
                              freq_scale, capacity, d_table, d_table ? n_table : 0);
}

// CudaDevice::qkv_postprocess_batch (cuda.rs:2478-2519; kernels.rs:1231-1330)
// without the Gemma-4 head norms, as mrml_hip_rope_kv_append_f16 is the
// single-token form: `batch` stacked q|k|v rows at positions start_pos + i,
// row i's K/V to cache row (cache_start + i) % capacity.
int mrml_hip_rope_kv_append_f16_batch(mrml_hip_ctx *ctx, float *qkv, uint16_t *k_cache, uint16_t *v_cache,
                                      int32_t start_pos, int32_t cache_start, int32_t batch, int32_t n_heads,
                                      int32_t n_kv_heads, int32_t head_dim, float freq_base, float freq_scale,
                                      int32_t capacity, int32_t k_format, int32_t v_format, const float *d_table,
                                      int32_t n_table)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, qkv && k_cache && v_cache, "rope_kv_append_f16_batch: null pointer");
    if (k_format < 0 || k_format > 2 || v_format < 0 || v_format > 2)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "rope_kv_append_f16_batch: k_format=%d v_format=%d (0 f16, 1 Q8_0, "
                    "2 Q4_0)", k_format, v_format);
    REQUIRE(ctx, n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && head_dim <= 1024,
            "rope_kv_append_f16_batch: n_heads=%d n_kv_heads=%d head_dim=%d", n_heads, n_kv_heads, head_dim);
    REQUIRE(ctx, (k_format == 0 && v_format == 0) || head_dim % 32 == 0,
            "rope_kv_append_f16_batch: quantised caches need head_dim %% 32 == 0 (head_dim=%d)", head_dim);
    // rows of one launch must not share a cache row
    REQUIRE(ctx, capacity > 0 && batch > 0 && batch <= capacity && batch <= 65535,
            "rope_kv_append_f16_batch: batch=%d capacity=%d (batch within 1..min(capacity, 65535))", batch,
            capacity);
    REQUIRE(ctx, start_pos >= 0 && cache_start >= 0 && start_pos <= INT32_MAX - batch &&
                     cache_start <= INT32_MAX - batch,
            "rope_kv_append_f16_batch: start_pos=%d cache_start=%d", start_pos, cache_start);
    REQUIRE(ctx, ((uintptr_t)d_table & 7) == 0 && n_table >= 0, "rope_kv_append_f16_batch: table");
    return launch_rope_kv_any(ctx, qkv, k_cache, v_cache, start_pos, n_heads, n_kv_heads, head_dim, freq_base,
                              freq_scale, capacity, d_table, d_table ? n_table : 0, batch, cache_start - start_pos,
                              k_format, v_format);
}

// CudaDevice::rope_256k (cuda.rs:2248-2285): rope_1d_batched (ops.rs:185-208)
// of n_heads contiguous heads in place, cos/sin from an optional table.
int mrml_hip_rope(mrml_hip_ctx *ctx, float *vec, int32_t pos, int32_t head_dim, int32_t n_heads, float freq_base,
                  float freq_scale, const float *d_table, int32_t n_table)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, vec, "rope: null pointer");
    REQUIRE(ctx, pos >= 0 && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && head_dim <= 1024,
            "rope: pos=%d n_heads=%d head_dim=%d", pos, n_heads, head_dim);
    REQUIRE(ctx, ((uintptr_t)d_table & 7) == 0 && n_table >= 0, "rope: table");
    return launch_rope(ctx, vec, pos, n_heads, head_dim, freq_base, freq_scale, d_table, d_table ? n_table : 0);
}

// CudaDevice::geglu / swiglu (cuda.rs:2182-2246): out = gelu_tanh(gate) * up,
// out = silu(gate) * up elementwise (ops.rs:107-130).
static int glu_args_ok(mrml_hip_ctx *ctx, const char *name, const float *gate, const float *up, const float *out,
                       int32_t n)
{
    REQUIRE(ctx, n >= 0 && n <= INT32_MAX - 255, "%s: n=%d", name, n);
    REQUIRE(ctx, n == 0 || (gate && up && out), "%s: null pointer", name);
    return MRML_HIP_OK;
}

int mrml_hip_geglu(mrml_hip_ctx *ctx, const float *gate, const float *up, float *out, int32_t n)
{
    CTX_GUARD(ctx);
    if (int rc = glu_args_ok(ctx, "geglu", gate, up, out, n)) return rc;
    return n ? launch_geglu_rows(ctx, gate, up, out, n) : MRML_HIP_OK;
}

int mrml_hip_swiglu(mrml_hip_ctx *ctx, const float *gate, const float *up, float *out, int32_t n)
{
    CTX_GUARD(ctx);
    if (int rc = glu_args_ok(ctx, "swiglu", gate, up, out, n)) return rc;
    return n ? launch_swiglu_rows(ctx, gate, up, out, n) : MRML_HIP_OK;
}

// CudaDevice::add (cuda.rs:2579-2593): out = a + b elementwise.
int mrml_hip_add(mrml_hip_ctx *ctx, const float *a, const float *b, float *out, int32_t n)
{
    CTX_GUARD(ctx);
    if (int rc = glu_args_ok(ctx, "add", a, b, out, n)) return rc;
    return n ? launch_add_rows(ctx, a, b, out, n) : MRML_HIP_OK;
}

// Arguments shared by the decode-attention entries: head_dim a multiple of
// 32 up to 512, groups of up to 16 query heads per kv head, cache formats
// 0 (f16), 1 (Q8_0), 2 (Q4_0) (KvCacheFormat::cuda_code, kv_cache.rs:16-22).
static int attn_args_ok(mrml_hip_ctx *ctx, const char *name, const float *q, const uint16_t *k_cache,
                        const uint16_t *v_cache, const float *out, const void *pack, int32_t n_past,
                        const int32_t *d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t capacity,
                        int32_t k_format = 0, int32_t v_format = 0)
{
    REQUIRE(ctx, q && k_cache && v_cache && (out || pack), "%s: null pointer or no output", name);
    if (k_format < 0 || k_format > 2 || v_format < 0 || v_format > 2)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "%s: k_format=%d v_format=%d (0 f16, 1 Q8_0, 2 Q4_0)", name,
                    k_format, v_format);
    REQUIRE(ctx, n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
            "%s: n_heads=%d n_kv_heads=%d", name, n_heads, n_kv_heads);
    REQUIRE(ctx, attn_any_ok(n_heads, n_kv_heads, head_dim),
            "%s: head_dim=%d (a multiple of 32 up to 512), group %d (at most 16)", name, head_dim,
            n_heads / n_kv_heads);
    REQUIRE(ctx, capacity > 0 && capacity <= attn_max_capacity() && (d_pos || n_past >= 0),
            "%s: n_past=%d capacity=%d (at most %d)", name, n_past, capacity, attn_max_capacity());
    REQUIRE(ctx, ((((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)q | (uintptr_t)pack) & 15) == 0),
            "%s: pointers must be 16-byte aligned", name);
    return MRML_HIP_OK;
}

static int attn_exact(mrml_hip_ctx *ctx, const float *q, const uint16_t *k_cache, const uint16_t *v_cache, float *out,
                      void *pack, int32_t n_past, const int32_t *d_pos, int32_t n_heads, int32_t n_kv_heads,
                      int32_t head_dim, float scale, int32_t capacity, int32_t sliding_window, int32_t k_format = 0,
                      int32_t v_format = 0)
{
    void *part = workspace(ctx, attn_scratch_bytes(n_heads, capacity));
    if (!part) return MRML_HIP_E_ALLOC;
    if (!attn_tuned(n_heads, n_kv_heads, head_dim, k_format, v_format))
        return launch_attn_any(ctx, q, 0, k_cache, v_cache, out, pack, d_pos, n_past, 1, n_heads, n_kv_heads,
                               head_dim, k_format, v_format, scale, capacity, part, sliding_window);
    return launch_attn_decode_f16(ctx, q, k_cache, v_cache, out, pack, d_pos, n_past, n_heads, n_kv_heads, scale,
                                  capacity, part, sliding_window);
}

// The split (flash-decoding) form serves the tuned shape; other head sizes,
// groups and formats run the exact form, which meets any tolerance.
static int attn_split(mrml_hip_ctx *ctx, const float *q, const uint16_t *k_cache, const uint16_t *v_cache, float *out,
                      void *pack, int32_t n_past, const int32_t *d_pos, int32_t n_heads, int32_t n_kv_heads,
                      int32_t head_dim, float scale, int32_t capacity, int32_t sliding_window, int32_t k_format = 0,
                      int32_t v_format = 0)
{
    if (!attn_tuned(n_heads, n_kv_heads, head_dim, k_format, v_format))
        return attn_exact(ctx, q, k_cache, v_cache, out, pack, n_past, d_pos, n_heads, n_kv_heads, head_dim, scale,
                          capacity, sliding_window, k_format, v_format);
    void *part = workspace(ctx, attn_split_scratch_bytes(n_heads, capacity));
    if (!part) return MRML_HIP_E_ALLOC;
    return launch_attn_split_f16(ctx, q, const_cast<uint16_t *>(k_cache), const_cast<uint16_t *>(v_cache), out, pack,
                                 d_pos, n_past, n_heads, n_kv_heads, scale, capacity, false, nullptr, 0, 0.0f, 0.0f,
                                 part, sliding_window);
}

int mrml_hip_attn_decode_f16(mrml_hip_ctx *ctx, const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                             float *out, void *pack, int32_t n_past, const int32_t *d_pos, int32_t n_heads,
                             int32_t n_kv_heads, int32_t head_dim, float scale, int32_t capacity)
{
    CTX_GUARD(ctx);
    if (int rc = attn_args_ok(ctx, "attn_decode_f16", q, k_cache, v_cache, out, pack, n_past, d_pos, n_heads,
                              n_kv_heads, head_dim, capacity))
        return rc;
    return attn_exact(ctx, q, k_cache, v_cache, out, pack, n_past, d_pos, n_heads, n_kv_heads, head_dim, scale,
                      capacity, -1);
}

int mrml_hip_attn_decode_f16_split(mrml_hip_ctx *ctx, const float *q, const uint16_t *k_cache,
                                   const uint16_t *v_cache, float *out, void *pack, int32_t n_past,
                                   const int32_t *d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                   float scale, int32_t capacity)
{
    CTX_GUARD(ctx);
    if (int rc = attn_args_ok(ctx, "attn_decode_f16_split", q, k_cache, v_cache, out, pack, n_past, d_pos, n_heads,
                              n_kv_heads, head_dim, capacity))
        return rc;
    return attn_split(ctx, q, k_cache, v_cache, out, pack, n_past, d_pos, n_heads, n_kv_heads, head_dim, scale,
                      capacity, -1);
}

// CudaDevice::attention_causal with its own argument list (cuda.rs:2658-2697),
// caches of any of the three formats.
int mrml_hip_attention_causal(mrml_hip_ctx *ctx, const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                              float *out, int32_t n_past, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                              float scale, int32_t sliding_window, int32_t capacity, int32_t k_format,
                              int32_t v_format)
{
    CTX_GUARD(ctx);
    if (int rc = attn_args_ok(ctx, "attention_causal", q, k_cache, v_cache, out, nullptr, n_past, nullptr, n_heads,
                              n_kv_heads, head_dim, capacity, k_format, v_format))
        return rc;
    return attn_exact(ctx, q, k_cache, v_cache, out, nullptr, n_past, nullptr, n_heads, n_kv_heads, head_dim, scale,
                      capacity, sliding_window, k_format, v_format);
}

// CudaDevice::attention_prefill (cuda.rs:2727-2770): `batch` queries at
// positions cache_start + i, query row i q_stride floats into q (the
// reference passes q.len() / batch), output rows of n_heads * head_dim.  Row
// i is bit-identical to mrml_hip_attention_causal at n_past = cache_start + i
// on the same caches (the K/V of every row already appended).
int mrml_hip_attention_prefill(mrml_hip_ctx *ctx, const float *q, int32_t q_stride, const uint16_t *k_cache,
                               const uint16_t *v_cache, float *out, int32_t cache_start, int32_t batch,
                               int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                               int32_t sliding_window, int32_t capacity, int32_t k_format, int32_t v_format)
{
    CTX_GUARD(ctx);
    if (int rc = attn_args_ok(ctx, "attention_prefill", q, k_cache, v_cache, out, nullptr, cache_start, nullptr,
                              n_heads, n_kv_heads, head_dim, capacity, k_format, v_format))
        return rc;
    REQUIRE(ctx, batch > 0 && cache_start <= INT32_MAX - batch, "attention_prefill: batch=%d cache_start=%d", batch,
            cache_start);
    REQUIRE(ctx, q_stride >= n_heads * head_dim, "attention_prefill: q_stride=%d below n_heads * head_dim = %d",
            q_stride, n_heads * head_dim);
    const size_t qd = (size_t)n_heads * head_dim;
    // rows per launch: scores of at most kPrefillScoreBytes, grid z within 65535
    const size_t per = attn_scratch_bytes(n_heads, capacity);
    const int rn = (int)std::max<size_t>(1, std::min<size_t>(std::min(batch, 65535), kPrefillScoreBytes / per));
    void *part = workspace(ctx, (size_t)rn * per);
    if (!part) return MRML_HIP_E_ALLOC;
    const bool tuned = attn_tuned(n_heads, n_kv_heads, head_dim, k_format, v_format);
    for (int r0 = 0; r0 < batch; r0 += rn) {
        const int n = std::min(rn, batch - r0);
        const int rc = tuned ? launch_attn_rows_f16(ctx, q + (size_t)r0 * q_stride, q_stride, k_cache, v_cache,
                                                    out + r0 * qd, cache_start + r0, n, n_heads, n_kv_heads, scale,
                                                    capacity, part, sliding_window)
                             : launch_attn_any(ctx, q + (size_t)r0 * q_stride, q_stride, k_cache, v_cache,
                                               out + r0 * qd, nullptr, nullptr, cache_start + r0, n, n_heads,
                                               n_kv_heads, head_dim, k_format, v_format, scale, capacity, part,
                                               sliding_window);
        if (rc) return rc;
    }
    return MRML_HIP_OK;
}

int mrml_hip_attention_causal_split(mrml_hip_ctx *ctx, const float *q, const uint16_t *k_cache,
                                    const uint16_t *v_cache, float *out, int32_t n_past, int32_t n_heads,
                                    int32_t n_kv_heads, int32_t head_dim, float scale, int32_t sliding_window,
                                    int32_t capacity, int32_t k_format, int32_t v_format)
{
    CTX_GUARD(ctx);
    if (int rc = attn_args_ok(ctx, "attention_causal_split", q, k_cache, v_cache, out, nullptr, n_past, nullptr,
                              n_heads, n_kv_heads, head_dim, capacity, k_format, v_format))
        return rc;
    return attn_split(ctx, q, k_cache, v_cache, out, nullptr, n_past, nullptr, n_heads, n_kv_heads, head_dim, scale,
                      capacity, sliding_window, k_format, v_format);
}

// ---- the Gemma-2-shape model --------------------------------------------------------

int mrml_hip_gemma2_create(mrml_hip_ctx *ctx, const mrml_hip_gemma2_config *cfg, const void *tok_embd,
                           const float *output_norm, const mrml_hip_gemma2_layer *layers, mrml_hip_gemma2 **out)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, cfg && tok_embd && output_norm && layers && out, "gemma2_create: null argument");
    *out = nullptr;
    if (int rc = check_model_config(ctx, *cfg)) return rc;
    const mrml_hip_gemma2_config &c = *cfg;
    for (int l = 0; l < c.n_layers; ++l) {
        const mrml_hip_gemma2_layer &L = layers[l];
        REQUIRE(ctx, L.wq && L.wk && L.wv && L.wo && L.w_gate && L.w_up && L.w_down && L.attn_norm &&
                         L.post_attn_norm && L.ffn_norm && L.post_ffw_norm,
                "gemma2_create: layer %d has a null tensor", l);
    }
    mrml_hip_gemma2 *m = new (std::nothrow) mrml_hip_gemma2;
    if (!m) return fail(ctx, MRML_HIP_E_ALLOC, "gemma2_create: out of host memory");
    m->cfg = c;
    m->tok_embd = tok_embd;
    m->output_norm = output_norm;
    m->layers.assign(layers, layers + c.n_layers);

    const size_t qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim;
    const size_t in_max = qd > (size_t)c.dim ? qd : (size_t)c.dim;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = align_up(off + bytes, 256);
        return at;
    };
    const size_t o_h = take(c.dim * 4), o_h2 = take(c.dim * 4), o_qkv = take((qd + 2 * kvd) * 4), o_o = take(c.dim * 4),
                 o_f = take(c.dim * 4), o_act = take((size_t)c.ffn_dim * 4), o_logits = take((size_t)c.vocab * 4),
                 o_xpack = take(act_pack_bytes((int)(in_max / 32))), o_apack = take(act_pack_bytes((int)(qd / 32))),
                 o_actpack = take(act_pack_bytes(c.ffn_dim / 32)),
                 o_part = take(std::max(attn_scratch_bytes(c.n_heads, c.ctx_len),
                                        c.numerics == MRML_HIP_NUMERICS_FAST
                                            ? attn_split_scratch_bytes(c.n_heads, c.ctx_len)
                                            : (size_t)0)),
                 o_argmax = take((size_t)argmax_parts(c.vocab) * 8), o_ring = take(recent_ring_bytes()),
                 o_select = take(vocab_select_scratch_bytes(c.vocab, kSamplerTopKMax)),
                 o_rope = take((size_t)c.ctx_len * c.head_dim * sizeof(float)),
                 o_freqs = take((size_t)c.head_dim / 2 * sizeof(float));
    hipError_t e = hipMalloc(&m->arena, off);
    if (e != hipSuccess) {
        delete m;
        return fail(ctx, MRML_HIP_E_ALLOC, "gemma2_create: hipMalloc(%zu): %s", off, hipGetErrorString(e));
    }
    uint8_t *base = (uint8_t *)m->arena;
    m->h = (float *)(base + o_h);
    m->h2 = (float *)(base + o_h2);
    m->qkv = (float *)(base + o_qkv);
    m->o = (float *)(base + o_o);
    m->f = (float *)(base + o_f);
    m->act = (float *)(base + o_act);
    m->logits = (float *)(base + o_logits);
    m->xpack = base + o_xpack;
    m->attn_pack = base + o_apack;
    m->act_pack = base + o_actpack;
    m->attn_part = base + o_part;
    m->argmax_scratch = base + o_argmax;
    m->recent_ring = base + o_ring;
    m->select_scratch = base + o_select;
    m->rope_table = (float *)(base + o_rope);
    m->rope_freqs = (float *)(base + o_freqs);
    e = hipMemset(m->recent_ring, 0xff, recent_ring_bytes());  // position -1: no entry
    if (e != hipSuccess) {
        (void)hipFree(m->arena);
        delete m;
        return fail(ctx, MRML_HIP_E_HIP, "gemma2_create: hipMemset: %s", hipGetErrorString(e));
    }
    int rc = fill_rope_table(ctx, m->rope_table, c.ctx_len, c.head_dim, c.rope_base, 1.0f);
    if (!rc) rc = fill_rope_freqs(ctx, m->rope_freqs, c.head_dim, c.rope_base);
    if (rc) {
        (void)hipFree(m->arena);
        delete m;
        return rc;
    }
    *out = m;
    return MRML_HIP_OK;
}

int mrml_hip_gemma2_destroy(mrml_hip_ctx *ctx, mrml_hip_gemma2 *m)
{
    CTX_GUARD(ctx);
    if (!m) return MRML_HIP_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(m->arena);
    if (m->pf_arena) (void)hipFree(m->pf_arena);
    delete m;
    return e == hipSuccess ? MRML_HIP_OK : hip_fail(ctx, e, "gemma2_destroy");
}

int mrml_hip_gemma2_step(mrml_hip_ctx *ctx, mrml_hip_gemma2 *m, int32_t *d_state, uint16_t *d_k_cache,
                         uint16_t *d_v_cache, float *d_logits, int32_t *d_argmax, int32_t *d_hist, int32_t hist_cap,
                         const int32_t *d_prompt, int32_t prompt_len)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, m && d_state && d_k_cache && d_v_cache, "gemma2_step: null argument");
    REQUIRE(ctx, (((uintptr_t)d_k_cache | (uintptr_t)d_v_cache | (uintptr_t)d_logits) & 15) == 0,
            "gemma2_step: caches and logits must be 16-byte aligned");
    const mrml_hip_gemma2_config &c = m->cfg;
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    const size_t layer_cache = (size_t)c.ctx_len * kvd;
    int32_t *d_token = d_state, *d_pos = d_state + 1;
    float *logits = d_logits ? d_logits : m->logits;
    int rc;
#define STEP(call)                      \
    do {                                \
        if ((rc = (call)) != 0) return rc; \
    } while (0)
    // With the fused instances (resnorm_shape), each sandwich residual runs
    // inside the matvec that consumes its norm: the post-attention one ahead
    // of gate/up, the post-FFN one ahead of the next block's q|k|v.  Every
    // workgroup there reads h while workgroup 0 writes the update, so h
    // alternates between two buffers (A -> B -> A per block) and ends in A.
    const bool fused = resnorm_shape(c.dim) && c.ffn_dim % 64 == 0;
    const bool fast = c.numerics == MRML_HIP_NUMERICS_FAST;
    const bool split_ffn = ffn_split_ok(c.dim, c.ffn_dim);
    float *hA = m->h, *hB = m->h2;
    STEP(launch_embedding(ctx, m->tok_embd, c.tie_type, d_token, 0, sqrtf((float)c.dim), hA,
                          m->layers[0].attn_norm, c.eps, nullptr, m->xpack, c.dim, c.vocab));
    for (int l = 0; l < c.n_layers; ++l) {
        const mrml_hip_gemma2_layer &L = m->layers[l];
        uint16_t *kc = d_k_cache + (size_t)l * layer_cache, *vc = d_v_cache + (size_t)l * layer_cache;
        const float *next_norm = l + 1 < c.n_layers ? m->layers[l + 1].attn_norm : m->output_norm;
        if (fused && l > 0)
            STEP(launch_qkv_resnorm(ctx, L.wq, L.wk, L.wv, m->f, m->layers[l - 1].post_ffw_norm, hB, hA, L.attn_norm,
                                    c.eps, m->qkv, qd, kvd, c.dim, fast));
        else
            STEP(launch_gemv_q4_0_qkv(ctx, L.wq, L.wk, L.wv, m->xpack, m->qkv, qd, kvd, c.dim));
        if (fast) {
            STEP(launch_attn_split_f16(ctx, m->qkv, kc, vc, nullptr, m->attn_pack, d_pos, 0, c.n_heads, c.n_kv_heads,
                                       c.attn_scale, c.ctx_len, true, m->rope_table, c.ctx_len, c.rope_base, 1.0f,
                                       m->attn_part, layer_window(c, l), m->rope_freqs));
        } else if (attn_rope_ok(c.n_heads, c.n_kv_heads)) {
            STEP(launch_attn_decode_rope_f16(ctx, m->qkv, kc, vc, nullptr, m->attn_pack, d_pos, 0, c.n_heads,
                                             c.n_kv_heads, c.attn_scale, c.ctx_len, m->rope_table, c.ctx_len,
                                             c.rope_base, 1.0f, m->attn_part, m->rope_freqs, layer_window(c, l)));
        } else {
            STEP(launch_rope_kv_f16(ctx, m->qkv, kc, vc, d_pos, 0, c.n_heads, c.n_kv_heads, c.head_dim, c.rope_base,
                                    1.0f, c.ctx_len, m->rope_table, c.ctx_len, 1, 0, m->rope_freqs));
            STEP(launch_attn_decode_f16(ctx, m->qkv, kc, vc, nullptr, m->attn_pack, d_pos, 0, c.n_heads,
                                        c.n_kv_heads, c.attn_scale, c.ctx_len, m->attn_part, layer_window(c, l)));
        }
        STEP(launch_gemv_q4_0(ctx, L.wo, m->attn_pack, m->o, c.dim, qd, fast));
        if (fused && split_ffn) {
            // the balanced split form: the GeGLU writes act and the pack blocks
            // it holds whole, the down projection quantises the rest from act
            STEP(launch_geglu_resnorm_split(ctx, L.w_gate, L.w_up, m->o, L.post_attn_norm, hA, hB, L.ffn_norm, c.eps,
                                            m->act, m->act_pack, c.ffn_dim, c.dim, fast));
        } else if (fused) {
            STEP(launch_geglu_resnorm(ctx, L.w_gate, L.w_up, m->o, L.post_attn_norm, hA, hB, L.ffn_norm, c.eps,
                                      m->act_pack, c.ffn_dim, c.dim, fast));
        } else {
            STEP(launch_residual_rms_norm(ctx, m->o, L.post_attn_norm, hA, hA, L.ffn_norm, c.eps, nullptr, m->xpack,
                                          c.dim, 1, fast));
            STEP(launch_gemv_q4_0_geglu_emit(ctx, L.w_gate, L.w_up, m->xpack, m->act, m->act_pack, c.ffn_dim,
                                             c.dim));
        }
        if (fused && split_ffn)
            STEP(launch_down_mix(ctx, L.w_down, m->act_pack, m->act, m->f, c.dim, c.ffn_dim));
        else
            STEP(launch_gemv_q4_0(ctx, L.w_down, m->act_pack, m->f, c.dim, c.ffn_dim, fast));
        if (!fused)
            STEP(launch_residual_rms_norm(ctx, m->f, L.post_ffw_norm, hA, hA, next_norm, c.eps, nullptr, m->xpack,
                                          c.dim, 1, fast));
        else if (l + 1 == c.n_layers)
            STEP(launch_residual_rms_norm(ctx, m->f, L.post_ffw_norm, hB, hA, next_norm, c.eps, nullptr, m->xpack,
                                          c.dim, 1, fast));
    }
    if (c.tie_type == MRML_HIP_Q4_0)
        STEP(launch_gemv_q4_0(ctx, m->tok_embd, m->xpack, logits, c.vocab, c.dim));
    else
        STEP(launch_gemv_q8_0(ctx, m->tok_embd, m->xpack, logits, c.vocab, c.dim, 0));
    if (m->sampler.top_k > 0) {
        const mrml_hip_sampler &sp = m->sampler;
        STEP(launch_vocab_select(ctx, logits, c.vocab, sp.d_valid, nullptr, 0, 0, MRML_HIP_SCORE_CPU, sp.temperature,
                                 0, sp.temperature > 0.0f ? sp.top_k : 1, d_argmax, nullptr, nullptr,
                                 m->select_scratch, d_state, m->recent_ring, 0, d_hist, hist_cap, d_prompt,
                                 prompt_len));
    } else {
        STEP(launch_argmax_step(ctx, logits, c.vocab, d_argmax, m->argmax_scratch, d_state, d_hist, hist_cap,
                                d_prompt, prompt_len, m->recent_ring));
    }
#undef STEP
    return MRML_HIP_OK;
}

// ---- prefill through the batched product ---------------------------------------

namespace {

// Tokens per chunk.  prefill_cuda's tile is 128 (model.rs:2395-2638); 512
// here gives the batched products four times the waves and streams the
// weights once per 512 tokens (2.1x the prefill rate at the Gemma-2-2B
// shape).  Results do not depend on it: every op keeps the token step's
// arithmetic.
constexpr int kPrefillChunk = 512;

// Attention rows per launch in a prefill chunk: the whole chunk unless its
// scores (n_heads * capacity floats a row) would pass kPrefillScoreBytes.
inline int prefill_attn_rows(const mrml_hip_gemma2_config &c)
{
    const size_t per = attn_scratch_bytes(c.n_heads, c.ctx_len);
    return (int)std::max<size_t>(1, std::min<size_t>(kPrefillChunk, kPrefillScoreBytes / per));
}

int prefill_buffers(mrml_hip_ctx *ctx, mrml_hip_gemma2 *m)
{
    if (m->pf_arena) return MRML_HIP_OK;
    const mrml_hip_gemma2_config &c = m->cfg;
    const size_t M = kPrefillChunk, qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim;
    const size_t widest = std::max<size_t>(std::max<size_t>(qd, c.dim), c.ffn_dim);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = align_up(off + bytes, 256);
        return at;
    };
    const size_t o_h = take(M * c.dim * 4), o_xn = take(M * c.dim * 4), o_qkv = take(M * (qd + 2 * kvd) * 4),
                 o_attn = take(M * qd * 4), o_o = take(M * c.dim * 4), o_gu = take(M * 2 * c.ffn_dim * 4),
                 o_f = take(M * c.dim * 4),
                 o_gp = take(gemm_pack_bytes((int32_t)widest, (int32_t)M)),
                 o_sc = take((size_t)prefill_attn_rows(c) * attn_scratch_bytes(c.n_heads, c.ctx_len));
    hipError_t e = hipMalloc(&m->pf_arena, off);
    if (e != hipSuccess) {
        m->pf_arena = nullptr;
        return fail(ctx, MRML_HIP_E_ALLOC, "gemma2_prefill: hipMalloc(%zu): %s", off, hipGetErrorString(e));
    }
    uint8_t *b = (uint8_t *)m->pf_arena;
    m->pf_h = (float *)(b + o_h), m->pf_xn = (float *)(b + o_xn), m->pf_qkv = (float *)(b + o_qkv);
    m->pf_attn = (float *)(b + o_attn), m->pf_o = (float *)(b + o_o), m->pf_gu = (float *)(b + o_gu);
    m->pf_f = (float *)(b + o_f);
    m->pf_gpack = b + o_gp;
    m->pf_scores = b + o_sc;
    return MRML_HIP_OK;
}

// Q8_0 of n rows of `cols` f32 values as a GEMM pack, then y = W * x for every row.
int gemm_rows(mrml_hip_ctx *ctx, mrml_hip_gemma2 *m, const void *w, const float *x, float *y, int rows, int cols, int n)
{
    if (int rc = launch_gemm_pack_quantize(ctx, x, m->pf_gpack, cols, n)) return rc;
    return launch_gemm_q4_0(ctx, w, m->pf_gpack, y, rows, cols, n, 0, m->cfg.numerics == MRML_HIP_NUMERICS_FAST);
}

}  // namespace

int mrml_hip_gemma2_reserve_prefill(mrml_hip_ctx *ctx, mrml_hip_gemma2 *m)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, m, "gemma2_reserve_prefill: null model");
    return prefill_buffers(ctx, m);
}

int mrml_hip_gemma2_prefill(mrml_hip_ctx *ctx, mrml_hip_gemma2 *m, const int32_t *d_tokens, int32_t n_tokens,
                            int32_t pos0, uint16_t *d_k_cache, uint16_t *d_v_cache, float *d_logits, int32_t *d_argmax)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, m && d_tokens && d_k_cache && d_v_cache, "gemma2_prefill: null argument");
    const mrml_hip_gemma2_config &c = m->cfg;
    REQUIRE(ctx, n_tokens > 0 && pos0 >= 0 && (int64_t)pos0 + n_tokens <= INT32_MAX,
            "gemma2_prefill: n_tokens=%d pos0=%d", n_tokens, pos0);
    REQUIRE(ctx, (((uintptr_t)d_k_cache | (uintptr_t)d_v_cache | (uintptr_t)d_logits) & 15) == 0,
            "gemma2_prefill: caches and logits must be 16-byte aligned");
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim, qkvd = qd + 2 * kvd;
    if (!(gemm_shape_ok(qd, c.dim, kPrefillChunk) && gemm_shape_ok(kvd, c.dim, kPrefillChunk) &&
          gemm_shape_ok(c.dim, qd, kPrefillChunk) && gemm_shape_ok(c.ffn_dim, c.dim, kPrefillChunk) &&
          gemm_shape_ok(c.dim, c.ffn_dim, kPrefillChunk)))
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "gemma2_prefill: a projection's shape does not fit the batched product");
    if (int rc = prefill_buffers(ctx, m)) return rc;
    const size_t layer_cache = (size_t)c.ctx_len * kvd;
    const float emb_scale = sqrtf((float)c.dim);
    const bool fast = c.numerics == MRML_HIP_NUMERICS_FAST;  // the one-FMA GEMM fold
    int rc;
#define STEP(call)                      \
    do {                                \
        if ((rc = (call)) != 0) return rc; \
    } while (0)
    for (int t0 = 0; t0 < n_tokens; t0 += kPrefillChunk) {
        const int n = std::min(kPrefillChunk, n_tokens - t0), p0 = pos0 + t0;
        float *h = m->pf_h, *xn = m->pf_xn;
        STEP(launch_embedding(ctx, m->tok_embd, c.tie_type, d_tokens + t0, 0, emb_scale, h, m->layers[0].attn_norm,
                              c.eps, xn, nullptr, c.dim, c.vocab, n));
        for (int l = 0; l < c.n_layers; ++l) {
            const mrml_hip_gemma2_layer &L = m->layers[l];
            uint16_t *kc = d_k_cache + (size_t)l * layer_cache, *vc = d_v_cache + (size_t)l * layer_cache;
            const float *next_norm = l + 1 < c.n_layers ? m->layers[l + 1].attn_norm : m->output_norm;
            // q, k, v of the chunk, stacked per token as the token step's q|k|v
            // (the pack of xn: the previous layer's norm writes it)
            if (l == 0) STEP(launch_gemm_pack_quantize(ctx, xn, m->pf_gpack, c.dim, n));
            {
                const void *qkv_w[3] = {L.wq, L.wk, L.wv};
                const int32_t qkv_rows[3] = {qd, kvd, kvd};
                STEP(launch_gemm_q4_0_stacked(ctx, qkv_w, qkv_rows, 3, m->pf_gpack, m->pf_qkv, c.dim, n, qkvd, fast));
            }
            if ((int64_t)p0 + n > c.ctx_len) {
                // The chunk wraps the ring: a later token's K/V row replaces
                // a position an earlier token still attends to, so each token
                // appends and attends in turn, as its token step does.
                for (int i = 0; i < n; ++i) {
                    float *qi = m->pf_qkv + (size_t)i * qkvd;
                    STEP(launch_rope_kv_f16(ctx, qi, kc, vc, nullptr, p0 + i, c.n_heads, c.n_kv_heads, c.head_dim,
                                            c.rope_base, 1.0f, c.ctx_len, m->rope_table, c.ctx_len, 1, 0,
                                            m->rope_freqs));
                    STEP(launch_attn_rows_f16(ctx, qi, (int)qkvd, kc, vc, m->pf_attn + (size_t)i * qd, p0 + i, 1,
                                              c.n_heads, c.n_kv_heads, c.attn_scale, c.ctx_len, m->pf_scores,
                                              layer_window(c, l)));
                }
            } else {
                // every token's rotated k and v enter the cache before any token
                // attends; token i then reads positions <= p0 + i only
                STEP(launch_rope_kv_f16(ctx, m->pf_qkv, kc, vc, nullptr, p0, c.n_heads, c.n_kv_heads, c.head_dim,
                                        c.rope_base, 1.0f, c.ctx_len, m->rope_table, c.ctx_len, n, 0,
                                        m->rope_freqs));
                for (int r0 = 0, rn = prefill_attn_rows(c); r0 < n; r0 += rn)
                    STEP(launch_attn_rows_f16(ctx, m->pf_qkv + (size_t)r0 * qkvd, (int)qkvd, kc, vc,
                                              m->pf_attn + (size_t)r0 * qd, p0 + r0, std::min(rn, n - r0),
                                              c.n_heads, c.n_kv_heads, c.attn_scale, c.ctx_len, m->pf_scores,
                                              layer_window(c, l)));
            }
            STEP(gemm_rows(ctx, m, L.wo, m->pf_attn, m->pf_o, c.dim, qd, n));
            STEP(launch_residual_rms_norm(ctx, m->pf_o, L.post_attn_norm, h, h, L.ffn_norm, c.eps, xn, nullptr, c.dim,
                                          n, fast, m->pf_gpack));
            // gate and up in one launch: token rows of g|u
            const void *gu_w[2] = {L.w_gate, L.w_up};
            const int32_t gu_rows[2] = {c.ffn_dim, c.ffn_dim};
            STEP(launch_gemm_q4_0_stacked(ctx, gu_w, gu_rows, 2, m->pf_gpack, m->pf_gu, c.dim, n, 0, fast));
            // act = gelu_tanh(g) * u per element (the GeGLU epilogue of the
            // matvec kernels, so each act value has the token step's bits),
            // quantized into the down projection's pack as it is formed
            STEP(launch_gemm_pack_geglu(ctx, m->pf_gu, m->pf_gu + c.ffn_dim, 2 * c.ffn_dim, m->pf_gpack, c.ffn_dim,
                                        n));
            STEP(launch_gemm_q4_0(ctx, L.w_down, m->pf_gpack, m->pf_f, c.dim, c.ffn_dim, n, 0, fast));
            STEP(launch_residual_rms_norm(ctx, m->pf_f, L.post_ffw_norm, h, h, next_norm, c.eps, xn, nullptr, c.dim,
                                          n, fast, l + 1 < c.n_layers ? m->pf_gpack : nullptr));
        }
        if (t0 + n < n_tokens) continue;
        // the last token's logits and greedy pick (the LM head of its token step)
        STEP(launch_quantize_q8_0(ctx, xn + (size_t)(n - 1) * c.dim, nullptr, m->xpack, c.dim));
        float *logits = d_logits ? d_logits : m->logits;
        if (c.tie_type == MRML_HIP_Q4_0)
            STEP(launch_gemv_q4_0(ctx, m->tok_embd, m->xpack, logits, c.vocab, c.dim));
        else
            STEP(launch_gemv_q8_0(ctx, m->tok_embd, m->xpack, logits, c.vocab, c.dim, 0));
        // the prompt's last 32 tokens enter the recent-token history
        STEP(launch_recent_ring_write(ctx, m->recent_ring, d_tokens, n_tokens, pos0));
        if (d_argmax && m->sampler.top_k > 0) {
            // the pick after a prompt: no token generated yet, state.pos = pos0 + n_tokens
            const mrml_hip_sampler &sp = m->sampler;
            STEP(launch_vocab_select(ctx, logits, c.vocab, sp.d_valid, nullptr, 0, 0, MRML_HIP_SCORE_CPU,
                                     sp.temperature, (uint64_t)pos0 + n_tokens, sp.temperature > 0.0f ? sp.top_k : 1,
                                     d_argmax, nullptr, nullptr, m->select_scratch, nullptr, m->recent_ring,
                                     (long long)pos0 + n_tokens - 1, nullptr, 0, nullptr, 0));
        } else if (d_argmax) {
            // the model's own argmax scratch, as in the token step: the
            // context workspace could be reallocated (and a captured graph
            // left pointing at freed memory)
            STEP(launch_argmax_step(ctx, logits, c.vocab, d_argmax, m->argmax_scratch, nullptr, nullptr, 0, nullptr,
                                    0, nullptr));
        }
    }
#undef STEP
    return MRML_HIP_OK;
}

int mrml_hip_gemma2_set_sampler(mrml_hip_ctx *ctx, mrml_hip_gemma2 *m, const mrml_hip_sampler *sampler)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, m, "gemma2_set_sampler: null model");
    if (!sampler) {
        m->sampler = mrml_hip_sampler{};
        return MRML_HIP_OK;
    }
    REQUIRE(ctx, sampler->top_k >= 1 && sampler->top_k <= kSamplerTopKMax,
            "gemma2_set_sampler: top_k=%d outside 1..%d", sampler->top_k, kSamplerTopKMax);
    REQUIRE(ctx, sampler->temperature == sampler->temperature, "gemma2_set_sampler: temperature is NaN");
    m->sampler = *sampler;
    return MRML_HIP_OK;
}

int mrml_hip_gemma2_activations(mrml_hip_ctx *ctx, mrml_hip_gemma2 *m, float **d_h, float **d_logits)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, m, "gemma2_activations: null model");
    if (d_h) *d_h = m->h;
    if (d_logits) *d_logits = m->logits;
    return MRML_HIP_OK;
}

}  // extern "C"
