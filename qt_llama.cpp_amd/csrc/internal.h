// internal.h -- host-side internals shared by the backend's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/mrml_hip.h"

struct mrml_hip_ctx {
    int32_t device = 0;
    hipStream_t stream = nullptr;
    hipDeviceProp_t props{};
    void *ws = nullptr;     // scratch: activation packs and partial results
    size_t ws_bytes = 0;
    void *noalloc_scratch = nullptr;  // the device's copy of the allocation-free GEMM's scratch
    std::string err;
};

namespace mrml {

// Record a failure on the context and return `code`.
int fail(mrml_hip_ctx *ctx, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
// Record a HIP error (with the call that produced it) and return MRML_HIP_E_HIP.
int hip_fail(mrml_hip_ctx *ctx, hipError_t e, const char *what);
// Make hipSetDevice(ctx->device) current; returns 0 or an error code.
int enter(mrml_hip_ctx *ctx);
// Check the launch that just happened.
int check_launch(mrml_hip_ctx *ctx, const char *kernel);
// Ensure at least `bytes` of scratch; returns its device pointer or null on failure.
void *workspace(mrml_hip_ctx *ctx, size_t bytes);

__host__ __device__ inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Launchers implemented in the kernel translation units.  All return 0 or a
// negative status and assume arguments were validated by the ABI layer.
int launch_quantize_q8_0(mrml_hip_ctx *ctx, const float *x, void *gguf, void *pack, int32_t n);
int launch_repack_q4_0(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols);
int launch_repack_q8_0(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols);
int launch_repack_q4_k(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols);
int launch_zero(mrml_hip_ctx *ctx, void *dst, size_t bytes);
int launch_copy(mrml_hip_ctx *ctx, void *dst, const void *src, size_t bytes);

// Q4_0 x Q8_0 matvec family; `xpack` is an activation pack for `cols`.
// relaxed: the tolerance path's balanced rows kernel where it pays (the
// f32 sum of a row in tree order, within 1e-5 of the block-ordered one)
int launch_gemv_q4_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y,
                     int32_t rows, int32_t cols, bool relaxed = false);
int launch_gemv_q4_0_gguf(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y,
                          int32_t rows, int32_t cols);
// f32-input forms: quantise x inside the kernel where a fixed instance exists.
bool ffn_split_ok(int dim, int ffn);
int launch_ffn_split(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *wd, const float *x, float *act,
                     void *pack, float *y, int32_t dim, int32_t ffn);
int split_main_blocks(int ffn);
// wd (nullable): the down projection that follows, whose rows the GeGLU's
// staging waves read ahead into the caches (when it runs nine rows a
// workgroup); results do not depend on it.
int launch_geglu_split(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act, void *pack,
                       int32_t rows, int32_t cols, const void *wd = nullptr);
// The split GeGLU with the post-attention sandwich residual fused ahead
// (h_out = h_in + rms_norm(t, w_post), then rms_norm(h_out, w_norm) as its
// input): act and the pack blocks launch_geglu_split writes.
int launch_geglu_resnorm_split(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *t,
                               const float *w_post, const float *h_in, float *h_out, const float *w_norm, float eps,
                               float *act, void *pack, int32_t rows, int32_t cols, bool fast);
int launch_down_mix(mrml_hip_ctx *ctx, const void *wd, const void *pack, const float *act, float *y, int32_t rows,
                    int32_t cols);
int launch_gemv_q4_0_x(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows, int32_t cols);
int launch_gemv_q4_0_geglu_x(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act,
                             void *act_pack, int32_t rows, int32_t cols);
int launch_gemv_q4_0_qkv_x(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const float *x,
                           float *y, int32_t q_rows, int32_t kv_rows, int32_t cols);
int launch_gemv_q4_0_geglu(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *xpack,
                           float *act, int32_t rows, int32_t cols);
int launch_gemv_q4_0_qkv(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv,
                         const void *xpack, float *y, int32_t q_rows, int32_t kv_rows,
                         int32_t cols);
int launch_gemv_q8_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y,
                     int32_t rows, int32_t cols, int32_t softcap);
int launch_gemv_q4_k(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y,
                     int32_t rows, int32_t cols);
int launch_argmax_f32(mrml_hip_ctx *ctx, const float *x, int32_t n, int32_t *out);
// act[i] = gelu_tanh(g[i]) * u[i] for i < n (the matvec kernels' GeGLU epilogue).
int launch_geglu_rows(mrml_hip_ctx *ctx, const float *g, const float *u, float *act, int n);
int launch_swiglu_rows(mrml_hip_ctx *ctx, const float *g, const float *u, float *act, int n);
int launch_add_rows(mrml_hip_ctx *ctx, const float *a, const float *b, float *out, int n);
// GeGLU over an activation pack that also writes the Q8_0 pack of its rows
// outputs (act nullable).
int launch_gemv_q4_0_geglu_emit(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *xpack, float *act,
                                void *act_pack, int32_t rows, int32_t cols);

// Batched Q4_0 x Q8_0 products with int8 MFMA.  The kernel reads its
// activations from a GEMM pack (token groups of 32 in MFMA lane order,
// gemm_pack_bytes), written from f32 rows [batch][cols] or converted from an
// activation pack of batch*cols values; y is [batch][rows].
bool gemm_shape_ok(int32_t rows, int32_t cols, int32_t batch);
size_t gemm_pack_bytes(int32_t cols, int32_t batch);
int launch_gemm_pack_quantize(mrml_hip_ctx *ctx, const float *x, void *gpack, int32_t cols, int32_t batch);
// The GEMM pack of act = gelu_tanh(g) * u (batch rows of `cols` values each,
// token rows `ld` floats apart in g and u), without act itself written.
int launch_gemm_pack_geglu(mrml_hip_ctx *ctx, const float *g, const float *u, int32_t ld, void *gpack,
                           int32_t cols, int32_t batch);
int launch_gemm_pack_from_act(mrml_hip_ctx *ctx, const void *pack, void *gpack, int32_t cols, int32_t batch);
// The allocation-free GEMM's file-scope device scratch: its size, and its
// address on the context's device (resolved once per device; 0 or a status).
size_t gemm_noalloc_scratch_bytes();
int gemm_noalloc_scratch(mrml_hip_ctx *ctx, void **out);
// y row stride ldy floats (0: rows; a multiple of 4, y 16-byte aligned)
int launch_gemm_q4_0(mrml_hip_ctx *ctx, const void *w, const void *gpack, float *y, int32_t rows, int32_t cols,
                     int32_t batch, int32_t ldy = 0, bool relaxed = false);
int launch_gemm_q4_0_stacked(mrml_hip_ctx *ctx, const void *const *w, const int32_t *rows, int n, const void *gpack,
                             float *y, int32_t cols, int32_t batch, int32_t ldy, bool relaxed = false);

// Argmax whose final pass can also advance a device-side decode loop
// (state = {token, pos}) and record the processed token in the recent-token
// ring (nullable); scratch holds argmax_parts(n) * 8 bytes.
int argmax_parts(int32_t n);
int launch_argmax_step(mrml_hip_ctx *ctx, const float *x, int32_t n, int32_t *out, void *scratch, int32_t *state,
                       int32_t *hist, int hist_cap, const int32_t *prompt, int prompt_len, void *ring);

// Vocabulary scoring (model.rs:2842-2907, kernels.rs:1085-1228): candidates
// are the valid ids minus 1, 2, 105, 106 while fewer than 4 tokens were
// generated; scoring 0 (CPU path) softcaps the raw logits with 30*tanh(x/30)
// and subtracts 3.5 once from recent ids, scoring 1 (device path) takes
// softcapped logits and subtracts 1.8 per occurrence; NaN scores drop out;
// ranks are by score, equal scores by lowest id.
//
// launch_vocab_topk: CudaDevice::vocab_topk's output (scoring 1), each of
// `parts` partitions' k best (score, id), (-inf, -1) past its candidates.
// scratch: vocab_topk_scratch_bytes.
//
// launch_vocab_select: the pick itself over the whole vocabulary (partitions
// of 2048 ids, then one merge): temperature <= 0 -> the best; else the
// CPU path's softmax draw over the k best with its LCG at position pos.
// out_token / out_scores / out_ids nullable (k entries, -inf / -1 past the
// candidates).  scratch: vocab_select_scratch_bytes.  The recent ids come
// from `recent`, or with ring from the ring of {position, token} (the last
// 32 positions up to cur = state[1] or host_cur).  With state (decode loop)
// the generated count is cur - (prompt_len - 1), pos is cur + 1, and the
// merge advances the loop like launch_argmax_step.
int vocab_parts(int32_t vocab);
size_t vocab_select_scratch_bytes(int32_t vocab, int32_t k);
bool vocab_select_ok(int32_t vocab, int32_t k);
int vocab_topk_chunks(int32_t vocab, int32_t parts);
bool vocab_topk_ok(int32_t vocab, int32_t k, int32_t parts);
size_t vocab_topk_scratch_bytes(int32_t vocab, int32_t k, int32_t parts);
size_t recent_ring_bytes();
int launch_recent_ring_write(mrml_hip_ctx *ctx, void *ring, const int32_t *tokens, int n, int pos0);
int launch_vocab_topk(mrml_hip_ctx *ctx, const float *logits, const uint8_t *valid, const int32_t *recent,
                      float *out_scores, int32_t *out_ids, int32_t vocab, int32_t n_recent, int32_t generated_count,
                      int32_t k, int32_t parts, void *scratch);
int launch_vocab_select(mrml_hip_ctx *ctx, const float *logits, int32_t vocab, const uint8_t *valid,
                        const int32_t *recent, int32_t n_recent, int32_t generated_count, int32_t scoring,
                        float temperature, uint64_t pos, int32_t k, int32_t *out_token, float *out_scores,
                        int32_t *out_ids, void *scratch, int32_t *state, void *ring, long long host_cur, int32_t *hist,
                        int hist_cap, const int32_t *prompt, int prompt_len);

// The Gemma-2 residual (h_out = h_in + rms_norm(t, w_post), then the next
// norm with w_norm) fused ahead of the gate/up GeGLU or the q|k|v matvec
// (gemv_q4_0.hip); h_out must not alias h_in.
bool resnorm_shape(int cols);
// fast: the decode step's tolerance path (tree sums for both norms).
int launch_geglu_resnorm(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *t, const float *w_post,
                         const float *h_in, float *h_out, const float *w_norm, float eps, void *act_pack, int32_t rows,
                         int32_t cols, bool fast = false);
int launch_qkv_resnorm(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const float *t,
                       const float *w_post, const float *h_in, float *h_out, const float *w_norm, float eps, float *y,
                       int32_t q_rows, int32_t kv_rows, int32_t cols, bool fast = false);

// ---- decode-step ops (decode.hip) --------------------------------------------
bool norm_dim_ok(int dim);
// rows > 1: rows consecutive vectors of dim values (out only, no pack)
int launch_rms_norm(mrml_hip_ctx *ctx, const float *x, const float *w, float eps, float *out, void *pack, int dim,
                    int rows = 1);
// fast: the tolerance path's tree-order sums (dims of one float4 per thread)
int launch_residual_rms_norm(mrml_hip_ctx *ctx, const float *t, const float *w_post, const float *h_in, float *h_out,
                             const float *w_next, float eps, float *xn, void *pack, int dim, int rows = 1,
                             bool fast = false, void *gpack = nullptr);
int launch_embedding(mrml_hip_ctx *ctx, const void *table, int type, const int32_t *d_token, int token, float scale,
                     float *h, const float *w_norm, float eps, float *xn, void *pack, int dim, int vocab,
                     int rows = 1);
int launch_rope_kv_f16(mrml_hip_ctx *ctx, float *qkv, uint16_t *k_cache, uint16_t *v_cache, const int32_t *d_pos,
                       int pos, int n_heads, int n_kv_heads, int head_dim, float base, float freq_scale, int capacity,
                       const float *table, int n_table, int rows = 1, int cache_shift = 0,
                       const float *freqs = nullptr);
// RoPE of n_heads contiguous heads of vec in place at one position.
int launch_rope(mrml_hip_ctx *ctx, float *vec, int pos, int n_heads, int head_dim, float base, float freq_scale,
                const float *table, int n_table, const float *freqs = nullptr);
// RoPE angles of the kernels above: (cos, sin) from `table` for positions <
// n_table; else from `freqs` (powf(base, 2i/d) per pair, host libm) with
// the host libm's cosf/sinf algorithm; else in double precision.  The
// pair values of fill_rope_freqs give every position the host's bits.
int fill_rope_freqs(mrml_hip_ctx *ctx, float *d_freqs, int head_dim, float base);
int attn_head_dim();
int attn_max_capacity();
// The attended window's limit: the capacity, or a sliding window below it
// (sliding_window <= 0: none).
int attn_window_limit(int capacity, int sliding_window);
size_t attn_scratch_bytes(int n_heads, int capacity);
// Streaming read of `bytes` (16-byte aligned) into nothing (sink: 1 KiB, rarely written).
int launch_read(mrml_hip_ctx *ctx, const void *src, size_t bytes, void *sink);
int launch_attn_decode_f16(mrml_hip_ctx *ctx, const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                           float *out, void *pack, const int32_t *d_pos, int n_past, int n_heads, int n_kv_heads,
                           float scale, int capacity, void *scratch, int sliding_window = -1);
bool attn_rope_ok(int n_heads, int n_kv_heads);
// `rows` batched queries at positions n_past0.., query rows q_stride floats
// apart (prefill); scratch of rows * attn_scratch_bytes(n_heads, capacity).
// Groups of up to 8 query heads per kv head.
int launch_attn_rows_f16(mrml_hip_ctx *ctx, const float *q, int q_stride, const uint16_t *k_cache,
                         const uint16_t *v_cache, float *out, int n_past0, int rows, int n_heads, int n_kv_heads,
                         float scale, int capacity, void *scratch, int sliding_window = -1);
// Attention over caches of any head size (a multiple of 32 up to 512),
// groups of up to 16 and the KV formats 0 (f16), 1 (Q8_0), 2 (Q4_0):
// `rows` queries at positions n_past0.. (or d_pos, rows = 1), the arithmetic
// of the CPU loop over KvCacheRow::dot_head / add_head_scaled.  scratch of
// rows * attn_scratch_bytes(n_heads, capacity).
bool attn_any_ok(int n_heads, int n_kv_heads, int head_dim);
bool attn_tuned(int n_heads, int n_kv_heads, int head_dim, int k_fmt, int v_fmt);
int launch_attn_any(mrml_hip_ctx *ctx, const float *q, int q_stride, const void *k_cache, const void *v_cache,
                    float *out, void *pack, const int32_t *d_pos, int n_past0, int rows, int n_heads, int n_kv_heads,
                    int head_dim, int k_fmt, int v_fmt, float scale, int capacity, void *scratch,
                    int sliding_window = -1);
// RoPE of `rows` stacked q|k|v rows at positions pos.. and their K/V appended
// to caches of formats k_fmt / v_fmt at cache rows (pos + i + cache_shift) %
// capacity (f16 caches: launch_rope_kv_f16 alone).
int launch_rope_kv_any(mrml_hip_ctx *ctx, float *qkv, void *k_cache, void *v_cache, int pos, int n_heads,
                       int n_kv_heads, int head_dim, float base, float freq_scale, int capacity, const float *table,
                       int n_table, int rows, int cache_shift, int k_fmt, int v_fmt, const float *freqs = nullptr);
int launch_attn_decode_rope_f16(mrml_hip_ctx *ctx, const float *qkv, uint16_t *k_cache, uint16_t *v_cache,
                                float *out, void *pack, const int32_t *d_pos, int n_past, int n_heads, int n_kv_heads,
                                float scale, int capacity, const float *table, int n_table, float base,
                                float freq_scale, void *scratch, const float *freqs = nullptr,
                                int sliding_window = -1);

// Bounded LDS-counter waits (exact_sum.h), one pair of device words per
// translation unit that has them: polls >= 0 sets the poll limit, timeouts
// (nullable) takes and clears the count of waits given up.
hipError_t wait_guard_gemv(int polls, uint32_t *timeouts);
hipError_t wait_guard_decode(int polls, uint32_t *timeouts);

// Split-K decode attention, the decode step's tolerance path (decode.hip):
// tiles of 32 positions, then a merge that also writes the Q8_0 pack.  With
// rope, qkv is the raw stacked q|k|v vector (RoPE and the K/V append as in
// launch_attn_decode_rope_f16); without, the q of a token whose K/V rows are
// in the caches.  scratch: attn_split_scratch_bytes(n_heads, capacity).
// Query-head groups of at most 8.
int attn_split_tiles(int capacity);
size_t attn_split_scratch_bytes(int n_heads, int capacity);
int launch_attn_split_f16(mrml_hip_ctx *ctx, const float *qkv, uint16_t *k_cache, uint16_t *v_cache, float *out,
                          void *pack, const int32_t *d_pos, int n_past, int n_heads, int n_kv_heads, float scale,
                          int capacity, bool rope, const float *table, int n_table, float base, float freq_scale,
                          void *scratch, int sliding_window = -1, const float *freqs = nullptr);

// Which form of the C library's expf the host runs (glibc picks its FMA build
// on x86-64 CPUs with FMA and AVX2); the device reproduces the same one.
bool host_expf_fused();
// RoPE cos/sin table [n_pos][head_dim/2] of (cos, sin) pairs computed with the
// host C library (the functions the reference calls), uploaded to d_table.
int fill_rope_table(mrml_hip_ctx *ctx, float *d_table, int n_pos, int head_dim, float base, float freq_scale);

}  // namespace mrml

// Argument guards of the extern "C" entry points: a null context is
// E_INVALID; every entry point first makes the context's device current.
#define CTX_GUARD(ctx)                                      \
    do {                                                    \
        if (!(ctx)) return MRML_HIP_E_INVALID;              \
        int rc_ = ::mrml::enter(ctx);                       \
        if (rc_) return rc_;                                \
    } while (0)

#define REQUIRE(ctx, cond, ...)                                                     \
    do {                                                                            \
        if (!(cond)) return ::mrml::fail((ctx), MRML_HIP_E_INVALID, __VA_ARGS__);   \
    } while (0)
