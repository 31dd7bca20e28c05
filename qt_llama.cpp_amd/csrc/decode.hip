// decode.hip -- the ops that complete a batch-1 token step around the
// matvecs: token embedding, RMSNorm (fused with Q8_0 quantisation of its
// output and with the sandwich-norm residual add), RoPE with f16 KV append,
// and GQA decode attention over the f16 cache.
//
// Every op follows the reference's operation order, so a token step is
// bit-identical to the CPU path:
//  * sums the reference evaluates sequentially in f32 (the RMSNorm sum of
//    squares, ops.rs:24-79; the attention dot, softmax denominator and
//    weighted sum of values, model.rs:1457-1590 / ops.rs:133-158) are
//    evaluated sequentially here too: the parallel work (products, exps,
//    loads) is spread over the workgroup, the dependent chain of adds runs
//    in one wave;
//  * expf and tanhf reproduce the host C library's results (libm_f32.h);
//  * RoPE's cos/sin come from a table the host fills with its own libm
//    (mrml_hip_rope_table); without a table the kernel evaluates powf, cosf
//    and sinf in double and rounds once.
// The Q8_0 packs these ops emit use the quantiser rule of quant.rs:193-228.
//
// Positions and tokens can be read from device memory (d_pos / d_token) so a
// captured token step replays unchanged for every position.

#include <math.h>

#include "device.h"
#include "exact_sum.h"
#include "internal.h"
#include "norm_block.h"

namespace mrml {

namespace {

constexpr int kMaxChunks = 4;        // float4 chunks per thread: dim <= 16 * blockDim
constexpr int kNormMaxThreads = 768;  // keeps ~170 VGPRs per lane for the norm kernels
constexpr int kScoreP = 64;    // cache positions per score workgroup (one per lane)
constexpr int kAttnHD = 256;   // head_dim served by the attention kernels

// s = 0; s += v[i] for i = 0..n-1, each add rounded (v 16-byte aligned in
// LDS).  Every lane of the calling wave runs the same chain on broadcast LDS
// reads.  Two register batches alternate: one is added while the next one's
// reads are in flight, with no copies between them, so the chain runs at the
// latency of its dependent adds.
__device__ float seq_sum(const float *v, int n)
{
    constexpr int B = 8;  // float4 per batch
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    float s = 0.0f;
    const int nb = n / (4 * B);
    auto add_batch = [&](const float4 (&c)[B]) {
#pragma unroll
        for (int k = 0; k < B; ++k) {
            s += c[k].x;
            s += c[k].y;
            s += c[k].z;
            s += c[k].w;
        }
    };
    if (nb > 0) {
        float4 a[B], b[B];
#pragma unroll
        for (int k = 0; k < B; ++k) a[k] = v4[k];
        int i = 0;
        for (; i + 2 <= nb; i += 2) {
            // the batch after the last re-reads the last one (never added)
            const int nbx = (i + 1) * B;
#pragma unroll
            for (int k = 0; k < B; ++k) b[k] = v4[nbx + k];
            add_batch(a);
            const int nba = (i + 2 < nb ? i + 2 : i + 1) * B;
#pragma unroll
            for (int k = 0; k < B; ++k) a[k] = v4[nba + k];
            add_batch(b);
        }
        if (i < nb) add_batch(a);
    }
    for (int i = nb * 4 * B; i < n; ++i) s += v[i];
    return s;
}

// out = rms_norm(x, w) (CudaDevice::rms_norm, cuda.rs:2102-2180; CPU
// ops.rs:24-79), optionally also as a Q8_0 pack.  One workgroup.
template <int CH>
__global__ __launch_bounds__(kNormMaxThreads) void rms_norm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                        float eps, float *__restrict__ out,
                                                        uint8_t *__restrict__ pack, int dim)
{
    extern __shared__ __align__(16) float lds[];
    const int n4 = dim >> 2;
    x += (size_t)blockIdx.y * dim;  // row blockIdx.y of a batch (no pack then)
    if (out) out += (size_t)blockIdx.y * dim;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    float4 v[CH], wv[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        const int c = threadIdx.x + k * blockDim.x;
        v[k] = c < n4 ? x4[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    load_w(w, wv, n4);
    norm_store(v, rms_scale(block_seq_sum_sq(v, n4, lds), dim, eps), wv, w != nullptr, out, pack, n4);
}

// Sandwich-norm residual of a Gemma-2 block followed by the next block's
// pre-norm (the per-layer order of model.rs:1185-2260):
//   h_out = h_in + rms_norm(t, w_post)
//   xn    = rms_norm(h_out, w_next)   -> xn (nullable) and its Q8_0 pack (nullable)
// One workgroup; h_out may equal h_in.
// FAST (one float4 per thread only): the two sums in tree order, the
// tolerance path's norm.
// gpack (one float4 per thread, xn set): xn of the batch's `rows` rows also
// written as a GEMM pack, quantized as quantize_gemm_pack_kernel does; the
// grid covers the pack's 32-token groups and the pad rows write zeros.
template <int CH, bool FAST = false>
__global__ __launch_bounds__(kNormMaxThreads) void residual_rms_norm_kernel(const float *__restrict__ t,
                                                                 const float *__restrict__ w_post,
                                                                 const float *h_in, float *h_out,
                                                                 const float *__restrict__ w_next, float eps,
                                                                 float *__restrict__ xn, uint8_t *__restrict__ pack,
                                                                 int dim, uint8_t *__restrict__ gpack, int rows)
{
    extern __shared__ __align__(16) float lds[];
    const int n4 = dim >> 2;
    if (CH == 1 && gpack && (int)blockIdx.y >= rows) {
        if ((int)threadIdx.x < n4)
            gemm_pack_put(gpack, gemm_groups(rows), n4 >> 3, blockIdx.y, threadIdx.x >> 3, threadIdx.x & 7, 0u, 0.0f);
        return;
    }
    if (blockIdx.y) {  // row blockIdx.y of a batch (prefill; no pack)
        const size_t r = (size_t)blockIdx.y * dim;
        t += r;
        h_in += r;
        h_out += r;
        if (xn) xn += r;
    }
    if constexpr (CH == 1) {
        const ResidualOps ops = residual_load(t, w_post, h_in, (xn || pack) ? w_next : nullptr, n4);
        residual_norm1<false, FAST>(ops, w_post != nullptr, w_next != nullptr, eps, h_out, xn, pack, dim,
                                    *reinterpret_cast<mrml_xsum::Shared4 *>(lds));
        if (gpack) {
            // this thread's own chunk of xn, read back after its store
            const int c = threadIdx.x;
            const float4 o = c < n4 ? reinterpret_cast<const float4 *>(xn)[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            uint32_t dbits;
            int qs;
            const uint32_t q = q8_0_block8x4(o, dbits, qs);  // every lane takes part
            if (c < n4) gemm_pack_put(gpack, gemm_groups(rows), n4 >> 3, blockIdx.y, c >> 3, c & 7, q, f16_bits_to_f32(dbits));
        }
        return;
    }
    const float4 *t4 = reinterpret_cast<const float4 *>(t);
    const float4 *hi4 = reinterpret_cast<const float4 *>(h_in);
    float4 *ho4 = reinterpret_cast<float4 *>(h_out);
    const float4 *wp4 = reinterpret_cast<const float4 *>(w_post);
    const float4 one4 = make_float4(1.0f, 1.0f, 1.0f, 1.0f), zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // every operand's load is issued before the first sum
    float4 v[CH], hv[CH], wv[CH], wn[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        const int c = threadIdx.x + k * blockDim.x;
        const int cc = c < n4 ? c : 0;
        v[k] = c < n4 ? t4[cc] : zero4;
        hv[k] = hi4[cc];
        wv[k] = w_post ? wp4[cc] : one4;
    }
    if (xn || pack) load_w(w_next, wn, n4);
    const float s1 = rms_scale(block_seq_sum_sq(v, n4, lds), dim, eps);
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        const int c = threadIdx.x + k * blockDim.x;
        float4 tn = scale4(v[k], s1);
        if (w_post) tn = mul4(tn, wv[k]);
        const float4 hn = add4(hv[k], tn);
        if (c < n4) ho4[c] = hn;
        v[k] = c < n4 ? hn : zero4;
    }
    if (!xn && !pack) return;
    norm_store(v, rms_scale(block_seq_sum_sq(v, n4, lds), dim, eps), wn, w_next != nullptr, xn, pack, n4);
}

// Token embedding (CudaDevice::embedding_q8_0, cuda.rs:2625-2656; CPU
// model.rs:1164-1182 with the sqrt(dim) scale of model.rs:1201): h = the
// dequantised table row (backend Q4_0 or Q8_0 layout) times `scale`, each
// value (q * d) * scale.  With w_norm or pack set it also writes
// rms_norm(h, w_norm) as f32 (xn) and/or as a Q8_0 pack -- the first layer's
// pre-norm.
template <int CH>
__global__ __launch_bounds__(kNormMaxThreads) void embedding_kernel(const uint8_t *__restrict__ table, int type,
                                                         const int32_t *__restrict__ d_token, int token, float scale,
                                                         float *__restrict__ h, const float *__restrict__ w_norm,
                                                         float eps, float *__restrict__ xn,
                                                         uint8_t *__restrict__ pack, int dim, int vocab)
{
    extern __shared__ __align__(16) float lds[];
    if (blockIdx.y) {  // row blockIdx.y of a batch (prefill; no pack)
        const size_t r = (size_t)blockIdx.y * dim;
        if (d_token) d_token += blockIdx.y;
        h += r;
        if (xn) xn += r;
    }
    int tok = d_token ? *d_token : token;  // the weight loads below do not wait for it
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
    const int n4 = dim >> 2, nb = dim >> 5;
    const size_t nblk = (size_t)vocab * nb, row = (size_t)tok * nb;
    float4 v[CH], wv[CH];
    if (xn || pack) load_w(w_norm, wv, n4);
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        const int c_raw = threadIdx.x + k * blockDim.x;
        const int c = c_raw < n4 ? c_raw : n4 - 1;
        const int b = c >> 3, p = (c & 7) * 4;  // block, first value index within it
        float q[4], d;
        if (type == MRML_HIP_Q4_0) {
            const uint32_t word = *reinterpret_cast<const uint32_t *>(table + (row + b) * 16 + (p & 15));
            const int shift = p < 16 ? 0 : 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = (float)((int)((word >> (8 * e + shift)) & 15u) - 8);
            d = f16_bits_to_f32(reinterpret_cast<const uint16_t *>(table + nblk * 16)[row + b]);
        } else {
            const uint32_t word = *reinterpret_cast<const uint32_t *>(table + (row + b) * 32 + p);
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = (float)(int8_t)(word >> (8 * e));
            d = f16_bits_to_f32(reinterpret_cast<const uint16_t *>(table + nblk * 32)[row + b]);
        }
        const float4 o = make_float4((q[0] * d) * scale, (q[1] * d) * scale, (q[2] * d) * scale, (q[3] * d) * scale);
        if (c_raw < n4) reinterpret_cast<float4 *>(h)[c_raw] = o;
        v[k] = c_raw < n4 ? o : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if (!xn && !pack) return;
    norm_store(v, rms_scale(block_seq_sum_sq(v, n4, lds), dim, eps), wv, w_norm != nullptr, xn, pack, n4);
}

// Where a RoPE kernel takes its angles (ops.rs:185-208: theta = pos *
// freq_scale / powf(base, 2i/d) in f32, then cosf and sinf):
//  * table: (cosf, sinf) pairs [n_table][head_dim/2] from the host's libm,
//    for pos < n_table;
//  * else freqs: the powf values per pair from the host's libm, theta formed
//    here and cosf / sinf evaluated with the host libm's algorithm
//    (libm_f32.h), so every position gets the host's bits;
//  * else the same with powf in double precision, rounded once.  The host's
//    powf is not correctly rounded everywhere, so a pair's frequency may then
//    differ from it by one ulp: 6 of 13280 pairs over ten bases and eleven
//    head sizes, none at base 10000.
struct RopeArgs {
    const float *table;
    const float *freqs;
    int n_table;
    float base, freq_scale;
    int fused;  // the host libm's FMA build (host_expf_fused)
};

__host__ inline RopeArgs rope_args(const float *table, int n_table, float base, float freq_scale, const float *freqs)
{
    return RopeArgs{table, freqs, table ? n_table : 0, base, freq_scale, (int)host_expf_fused()};
}

__device__ __forceinline__ void rope_cs(const RopeArgs &r, int pos, int i, int head_dim, float &c, float &s)
{
    if (r.table && pos >= 0 && pos < r.n_table) {
        const float2 cs = reinterpret_cast<const float2 *>(r.table)[(size_t)pos * (head_dim >> 1) + i];
        c = cs.x;
        s = cs.y;
    } else if (r.freqs) {
        const float theta = (float)pos * r.freq_scale / r.freqs[i];
        c = mrml_libm::cosf(theta, r.fused != 0);
        s = mrml_libm::sinf(theta, r.fused != 0);
    } else {
        const float expo = (float)(2 * i) / (float)head_dim;
        const float freq = (float)pow((double)r.base, (double)expo);
        const float theta = (float)pos * r.freq_scale / freq;
        c = mrml_libm::cosf(theta, r.fused != 0);
        s = mrml_libm::sinf(theta, r.fused != 0);
    }
}

// RoPE (NeoX half split, ops.rs:185-208) on the q and k heads of a stacked
// [q | k | v] vector, then k and v appended to the f16 caches at the cache
// row of `pos` (round to nearest even, as the reference CUDA path stores its
// cache, kernels.rs:1300-1322).  Cache layout [capacity][n_kv_heads][head_dim];
// a position past the capacity wraps (kernels.rs:1307-1313).  Rotated q (and
// k) are written back into qkv.  Angles as RopeArgs says.  Grid: n_heads +
// 2*n_kv_heads workgroups of head_dim/2 threads.
__global__ __launch_bounds__(512) void rope_kv_f16_kernel(float *__restrict__ qkv, uint16_t *__restrict__ k_cache,
                                                          uint16_t *__restrict__ v_cache,
                                                          const int32_t *__restrict__ d_pos, int pos_arg,
                                                          int n_heads, int n_kv_heads, int head_dim,
                                                          RopeArgs rope, int capacity, int cache_shift)
{
    // row blockIdx.y of a batch of stacked q|k|v rows at consecutive
    // positions; its K/V enter cache row (position + cache_shift) % capacity
    const int pos = (d_pos ? *d_pos : pos_arg) + (int)blockIdx.y;
    qkv += (size_t)blockIdx.y * (n_heads + 2 * n_kv_heads) * head_dim;
    const int half = head_dim >> 1, i = threadIdx.x, g = blockIdx.x;
    const size_t kv_dim = (size_t)n_kv_heads * head_dim;
    const int cpos = pos + cache_shift;
    const size_t cache_row = (size_t)(capacity > 0 ? cpos % capacity : cpos) * kv_dim;
    if (g < n_heads + n_kv_heads) {
        float c, s;
        rope_cs(rope, pos, i, head_dim, c, s);
        float *v = qkv + (size_t)g * head_dim;
        const float v0 = v[i], v1 = v[i + half];
        const float r0 = v0 * c - v1 * s;
        const float r1 = v0 * s + v1 * c;
        v[i] = r0;
        v[i + half] = r1;
        if (g >= n_heads && k_cache) {  // null caches: rotation only (quantised caches append after)
            uint16_t *dst = k_cache + cache_row + (size_t)(g - n_heads) * head_dim;
            dst[i] = f32_to_f16_rne(r0);
            dst[i + half] = f32_to_f16_rne(r1);
        }
    } else if (v_cache) {
        const int vh = g - n_heads - n_kv_heads;
        const float *src = qkv + (size_t)(n_heads + n_kv_heads) * head_dim + (size_t)vh * head_dim;
        uint16_t *dst = v_cache + cache_row + (size_t)vh * head_dim;
        dst[i] = f32_to_f16_rne(src[i]);
        dst[i + half] = f32_to_f16_rne(src[i + half]);
    }
}

// ---- GQA decode attention (model.rs:1457-1590, kv_cache.rs:72-124,
// ops.rs:133-158; GPU kernels.rs:1374-1561) --------------------------------------
//
// The window is the last min(n_past + 1, capacity) cache positions, oldest
// first (cache row = position % capacity).  Query head h reads kv head
// h / (n_heads / n_kv_heads).

__device__ __forceinline__ size_t cache_row_of(int t, int capacity) { return (size_t)(capacity > 0 ? t % capacity : t); }

// The window: the last min(n_past + 1, limit) positions, limit = the cache
// capacity or, below it, the sliding window (cuda.rs:2658-2697 sliding_window;
// kernels.rs:1398-1404).  Cache rows stay position % capacity.
__device__ __forceinline__ void attn_window(const int32_t *d_pos, int n_past_arg, int limit, int &window, int &start)
{
    const int n_past = d_pos ? *d_pos : n_past_arg;
    const int count = n_past + 1;
    window = (limit > 0 && count > limit) ? limit : count;
    start = count - window;
}

// Scores: score[h][p] = (sum_d q_h[d] * k_{start+p}[d], from -0.0 in d
// order) * scale.  Workgroup (tile of 64 positions, kv head) with one wave per
// query head of the group: the K tile (64 rows x 512 B) is loaded with
// coalesced 16-byte loads into LDS (rows padded to 520 B so a wave's 8-byte
// reads of 64 different rows are conflict-free), then lane p of wave g runs
// the chain of position p for head g (q from LDS as broadcasts).  Workgroups
// past the window exit at once.
constexpr int kKRow = kAttnHD * 2 + 8;  // padded K row in LDS, bytes

__global__ __launch_bounds__(512) void attn_scores_kernel(const float *__restrict__ q,
                                                          const uint16_t *__restrict__ k_cache,
                                                          const int32_t *__restrict__ d_pos, int n_past_arg,
                                                          int n_heads, int n_kv_heads, float scale, int capacity, int wlimit,
                                                          float *__restrict__ scores, int q_stride)
{
    constexpr int HD = kAttnHD, P = kScoreP;
    __shared__ __align__(16) float q_s[8][HD];
    __shared__ __align__(16) uint8_t k_s[P * kKRow];
    // query row blockIdx.z of a batch (prefill): rows q_stride floats apart
    // at consecutive positions
    q += (size_t)blockIdx.z * q_stride;
    scores += (size_t)blockIdx.z * n_heads * capacity;
    n_past_arg += (int)blockIdx.z;
    int window, start;
    attn_window(d_pos, n_past_arg, wlimit, window, start);
    const int p0 = blockIdx.x * P;
    if (p0 >= window) return;
    const int kvh = blockIdx.y, G = n_heads / n_kv_heads, nt = G * 64, tid = threadIdx.x;
    const size_t kv_dim = (size_t)n_kv_heads * HD;
    // K tile: 64 rows x 32 chunks of 16 B, chunk c of row r at r*32 + c
    constexpr int kChunks = P * (HD * 2 / 16);
    for (int base = 0; base < kChunks; base += 16 * 64) {
        uint4 tmp[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int c = base + k * nt + tid;
            const int r = c >> 5, off = c & 31;
            const int pr = p0 + r < window ? p0 + r : window - 1;
            tmp[k] = c < kChunks ? reinterpret_cast<const uint4 *>(
                                       k_cache + cache_row_of(start + pr, capacity) * kv_dim + (size_t)kvh * HD)[off]
                                 : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int c = base + k * nt + tid;
            if (c < kChunks) {
                uint32_t *dst = reinterpret_cast<uint32_t *>(k_s + (c >> 5) * kKRow + (c & 31) * 16);
                dst[0] = tmp[k].x;
                dst[1] = tmp[k].y;
                dst[2] = tmp[k].z;
                dst[3] = tmp[k].w;
            }
        }
        if (16 * nt >= kChunks) break;
    }
    for (int i = tid; i < G * HD; i += nt) q_s[i / HD][i % HD] = q[(size_t)kvh * G * HD + i];
    __syncthreads();
    const int g = tid >> 6, p = tid & 63;
    const uint8_t *krow = k_s + p * kKRow;
    const float4 *qg = reinterpret_cast<const float4 *>(q_s[g]);
    float dot = -0.0f;
#pragma unroll 8
    for (int d4 = 0; d4 < HD / 4; ++d4) {
        const uint2 kw = *reinterpret_cast<const uint2 *>(krow + d4 * 8);
        const float4 qv = qg[d4];
        dot += qv.x * f16_bits_to_f32(kw.x & 0xffffu);
        dot += qv.y * f16_bits_to_f32(kw.x >> 16);
        dot += qv.z * f16_bits_to_f32(kw.y & 0xffffu);
        dot += qv.w * f16_bits_to_f32(kw.y >> 16);
    }
    if (p0 + p < window) scores[(size_t)(kvh * G + g) * capacity + p0 + p] = dot * scale;
}

// Scores with an optional RoPE in front (the decode step's fused form).
// Workgroup (tile of 64 positions, kv head), 256 threads; waves 0..G-1 run
// the chains of the G query heads of the group.
//  * The K tile (64 rows x 512 B) goes to LDS with one 16-byte store per
//    chunk, rows padded to 528 B (16-byte aligned, conflict-free 16-byte
//    reads of 64 rows).
//  * ROPE: q comes raw from the stacked q|k|v vector and is rotated here
//    (NeoX half split, ops.rs:185-208; cos/sin from the host table when pos <
//    n_table).  The workgroup whose tile holds the newest position rotates
//    that position's k, rounds it to f16 (round to nearest even, as the
//    cache stores it, kernels.rs:1300-1322), uses it for that row and
//    appends it and the position's v to the caches.  Without ROPE, q is the
//    rotated query and the caches are complete.
//  * Lane p of wave g: dot = -0.0 + q[0]*k_p[0] + ... in d order, each
//    product rounded (an fma with addend -0.0 on the f16 k converted inline
//    rounds exactly as the product does, signs of zero included).
constexpr int kKRow2 = kAttnHD * 2 + 16;  // padded K row in LDS, bytes

// Native 4 and 2 x 32-bit vectors: copies of HIP's uint4 struct lower to
// memcpy, which keeps an array of them in scratch memory instead of registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kScoreT = 256;              // threads per score workgroup


// ---- attention over caches of any head size and KV format ------------------------
//
// The tuned kernels around this section serve the Gemma-2 shape (head_dim
// 256, f16 rows).  These serve every head_dim that is a multiple of 32 up
// to 512, groups of up to 16 query heads per kv head, and the reference's
// three cache formats (KvCacheFormat::cuda_code, kv_cache.rs:16-31): 0 f16
// rows (round to nearest even), 1 Q8_0 and 2 Q4_0 blocks of 32 values along
// a head, [capacity][n_kv_heads][head_dim/32 blocks] of 34 or 18 bytes.
// The arithmetic is the CPU loop's (model.rs:1526-1547 over
// KvCacheRow::dot_head / add_head_scaled, kv_cache.rs:73-125).

// K/V of a batch of stacked q|k|v rows, k already rotated in place (by
// rope_kv_f16_kernel with null caches), stored in the caches' formats
// (KvCacheRow::from_f32, kv_cache.rs:54-71): f16 by rounding to nearest
// even, Q8_0 and Q4_0 by the reference quantisers (quant.rs:193-228,
// 372-389) over each head's blocks of 32.  Grid (2 * n_kv_heads, rows):
// workgroup x < n_kv_heads stores k head x, the rest the v heads; lanes
// 0-31 and 32-63 take one block each.  Row z goes to cache row
// (pos0 + z + cache_shift) % capacity.
template <int KF, int VF>
__global__ __launch_bounds__(64) void kv_append_any_kernel(const float *__restrict__ qkv, uint8_t *__restrict__ k_cache,
                                                           uint8_t *__restrict__ v_cache, int pos0, int n_heads,
                                                           int n_kv_heads, int head_dim, int capacity, int cache_shift)
{
    const int z = blockIdx.y, g = blockIdx.x, lane = threadIdx.x, l = lane & 31;
    const bool is_k = g < n_kv_heads;
    const int head = is_k ? g : g - n_kv_heads, fmt = is_k ? KF : VF, nb = head_dim / 32;
    // k heads follow the q heads and v heads follow the k heads
    const float *src = qkv + (size_t)z * (n_heads + 2 * n_kv_heads) * head_dim + (size_t)(n_heads + g) * head_dim;
    const size_t bb = fmt == 0 ? 64 : (fmt == 1 ? 34 : 18);
    const int cpos = pos0 + z + cache_shift;
    uint8_t *dst = (is_k ? k_cache : v_cache) + (size_t)(cpos % capacity) * n_kv_heads * nb * bb + (size_t)head * nb * bb;
    for (int b0 = 0; b0 < nb; b0 += 2) {  // uniform: every lane runs the block quantisers
        const int b = b0 + (lane >> 5);
        const float v = b < nb ? src[b * 32 + l] : 0.0f;
        uint8_t *blk = dst + (size_t)b * bb;
        if (fmt == 0) {
            if (b < nb) reinterpret_cast<uint16_t *>(blk)[l] = f32_to_f16_rne(v);
        } else if (fmt == 1) {
            uint32_t dbits;
            int qsum;
            const int qv = q8_0_block32(v, dbits, qsum);
            if (b < nb) {
                if (l == 0) *reinterpret_cast<uint16_t *>(blk) = (uint16_t)dbits;
                blk[2 + l] = (uint8_t)(int8_t)qv;
            }
        } else {
            uint32_t dbits;
            const int qv = q4_0_block32(v, dbits);
            const int hi = __shfl_down(qv, 16, 64);  // value l + 16 of the block (same 32-lane half for l < 16)
            if (b < nb) {
                if (l == 0) *reinterpret_cast<uint16_t *>(blk) = (uint16_t)dbits;
                if (l < 16) blk[2 + l] = (uint8_t)(qv | (hi << 4));
            }
        }
    }
}

// Scores over K rows of format KF: score[h][p] = dot_head(q_h, k_{start+p}) *
// scale, dot_head as kv_cache.rs:73-95 -- f16: -0.0 + q[0]*k[0] + ... in d
// order; Q8_0 / Q4_0: the block-ordered fold s = s + (float)isum_b * (d_k *
// d_q) over the head's blocks against quantize_f32_to_q8_0(q_h) (formed
// here, per head, with the reference quantiser).  Workgroup (tile of 64
// positions, kv head, query row): lane p owns position p0 + p and wave w
// the heads w, w + 4, ... of the group; the K tile is staged through LDS in
// passes of 128 dims (f16 rows as they are; quantised blocks re-laid as
// 4-byte-aligned quants plus f32 scales), every chain carried across passes
// in registers.  Dynamic LDS as attn_any_scores_lds says.
constexpr int kAnyP = 64;                   // positions per workgroup (one per lane)
constexpr int kAnyT = 256;                  // 4 waves
constexpr int kAnyCh = 128;                 // dims per pass (4 blocks)
constexpr int kAnyMaxG = 16, kAnyMaxHD = 512;
constexpr int kAnyHPT = kAnyMaxG / 4;       // heads per thread at most
constexpr int kAnyKRow = kAnyCh * 2 + 16;   // f16 tile row stride, bytes
constexpr int kAnyDS = 5;                   // scale row stride (floats) of a quantised tile

__host__ __device__ constexpr int any_quant_row(int kf) { return 4 * (kf == 2 ? 16 : 32) + 4; }  // quant bytes per tile row
inline size_t attn_any_scores_lds(int kf, int G, int HD)
{
    if (kf == 0) return (size_t)G * HD * 4 + (size_t)kAnyP * kAnyKRow;
    const size_t qpart = ((size_t)G * HD + (size_t)G * (HD / 32) * 8 + 15) / 16 * 16;
    return qpart + (size_t)kAnyP * any_quant_row(kf) + (size_t)kAnyP * kAnyDS * 4;
}

template <int KF>
__global__ __launch_bounds__(kAnyT) void attn_scores_any_kernel(const float *__restrict__ q,
                                                                const uint8_t *__restrict__ k_cache,
                                                                const int32_t *__restrict__ d_pos, int n_past_arg,
                                                                int n_heads, int n_kv_heads, int head_dim, float scale,
                                                                int capacity, int wlimit, float *__restrict__ scores,
                                                                int q_stride)
{
    extern __shared__ __align__(16) uint8_t lds_any[];
    q += (size_t)blockIdx.z * q_stride;
    scores += (size_t)blockIdx.z * n_heads * capacity;
    n_past_arg += (int)blockIdx.z;
    int window, start;
    attn_window(d_pos, n_past_arg, wlimit, window, start);
    const int p0 = blockIdx.x * kAnyP;
    if (p0 >= window) return;
    const int kvh = blockIdx.y, G = n_heads / n_kv_heads, HD = head_dim, nb = HD / 32, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    constexpr int BB = KF == 0 ? 64 : (KF == 1 ? 34 : 18);  // cache bytes per 32 values
    constexpr int QB = KF == 2 ? 16 : 32;                   // quant bytes per block in LDS
    constexpr int KQR = any_quant_row(KF);
    const size_t row_bytes = (size_t)n_kv_heads * nb * BB;
    const uint8_t *khead = k_cache + (size_t)kvh * nb * BB;
    const float *qg = q + (size_t)kvh * G * HD;
    // q of the group: f32 (f16 K) or its Q8_0 blocks (quants, scales, quant sums)
    float *q_s = reinterpret_cast<float *>(lds_any);
    int8_t *qq = reinterpret_cast<int8_t *>(lds_any);
    float *qd = reinterpret_cast<float *>(lds_any + (size_t)G * HD);
    int *qsm = reinterpret_cast<int *>(lds_any + (size_t)G * HD + (size_t)G * nb * 4);
    const size_t qpart = KF == 0 ? (size_t)G * HD * 4 : ((size_t)G * HD + (size_t)G * nb * 8 + 15) / 16 * 16;
    uint8_t *kt = lds_any + qpart;                                     // f16 tile, or the quants
    float *kd = reinterpret_cast<float *>(kt + (size_t)kAnyP * KQR);   // quantised: [64][kAnyDS] scales
    if constexpr (KF == 0) {
        for (int i = tid; i < G * HD; i += kAnyT) q_s[i] = qg[i];
    } else {
        for (int base = 0; base < G * HD; base += kAnyT) {  // uniform: all lanes run the block quantiser
            const int i = base + tid;
            const float v = i < G * HD ? qg[i] : 0.0f;
            uint32_t dbits;
            int qsum;
            const int qv = q8_0_block32(v, dbits, qsum);
            if (i < G * HD) {
                qq[i] = (int8_t)qv;
                if ((i & 31) == 0) {
                    qd[i >> 5] = f16_bits_to_f32(dbits);
                    qsm[i >> 5] = qsum;
                }
            }
        }
    }
    float acc[kAnyHPT];
#pragma unroll
    for (int j = 0; j < kAnyHPT; ++j) acc[j] = KF == 0 ? -0.0f : 0.0f;
    for (int c0 = 0; c0 < HD; c0 += kAnyCh) {
        const int cn = HD - c0 < kAnyCh ? HD - c0 : kAnyCh, cb = cn / 32;
        __syncthreads();  // the previous pass's reads are done (and q is staged)
        if constexpr (KF == 0) {
            const int cpr = cn / 8;  // 16-byte chunks per row
            for (int c = tid; c < kAnyP * cpr; c += kAnyT) {
                const int r = c / cpr, o = c - r * cpr;
                const int pr = p0 + r < window ? p0 + r : window - 1;
                const uint8_t *src = khead + cache_row_of(start + pr, capacity) * row_bytes + (size_t)c0 * 2;
                *reinterpret_cast<u32x4 *>(kt + r * kAnyKRow + o * 16) = reinterpret_cast<const u32x4 *>(src)[o];
            }
        } else {
            const int hpr = cb * BB / 2;  // halfwords per row
            for (int c = tid; c < kAnyP * hpr; c += kAnyT) {
                const int r = c / hpr, o = 2 * (c - r * hpr);
                const int pr = p0 + r < window ? p0 + r : window - 1;
                const uint8_t *src = khead + cache_row_of(start + pr, capacity) * row_bytes + (size_t)(c0 / 32) * BB;
                const uint16_t hv = *reinterpret_cast<const uint16_t *>(src + o);
                const int b = o / BB, rb = o - b * BB;
                if (rb == 0)
                    kd[r * kAnyDS + b] = f16_bits_to_f32(hv);
                else
                    *reinterpret_cast<uint16_t *>(kt + r * KQR + b * QB + rb - 2) = hv;
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kAnyHPT; ++j) {
            const int g = wave + 4 * j;
            if (g < G) {  // uniform per wave
                if constexpr (KF == 0) {
                    const float4 *qh = reinterpret_cast<const float4 *>(q_s + (size_t)g * HD + c0);
                    const u32x4 *krow = reinterpret_cast<const u32x4 *>(kt + lane * kAnyKRow);
                    float dot = acc[j];
                    for (int d8 = 0; d8 < cn / 8; ++d8) {
                        const u32x4 kw = krow[d8];
                        const float4 qa = qh[2 * d8], qb = qh[2 * d8 + 1];
                        const uint32_t w[4] = {kw.x, kw.y, kw.z, kw.w};
                        const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const float prod = qv[e] * f16_bits_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xffffu);
                            dot = dot + prod;
                        }
                    }
                    acc[j] = dot;
                } else {
                    float sacc = acc[j];
                    for (int b = 0; b < cb; ++b) {
                        const int gb = g * nb + c0 / 32 + b;  // the query's block
                        const uint32_t *kw = reinterpret_cast<const uint32_t *>(kt + lane * KQR + b * QB);
                        const uint32_t *qw = reinterpret_cast<const uint32_t *>(qq + (size_t)gb * 32);
                        int isum = 0;
                        if constexpr (KF == 1) {
#pragma unroll
                            for (int w = 0; w < 8; ++w) isum = sdot4(kw[w], qw[w], isum);
                        } else {
                            // (n - 8) . a = n . a - 8 * sum(a): low nibbles pair with a[0..15], high with a[16..31]
#pragma unroll
                            for (int w = 0; w < 4; ++w) {
                                isum = sdot4(kw[w] & 0x0F0F0F0Fu, qw[w], isum);
                                isum = sdot4((kw[w] >> 4) & 0x0F0F0F0Fu, qw[w + 4], isum);
                            }
                            isum -= 8 * qsm[gb];
                        }
                        const float term = (float)isum * (kd[lane * kAnyDS + b] * qd[gb]);
                        sacc = sacc + term;
                    }
                    acc[j] = sacc;
                }
            }
        }
    }
    if (p0 + lane < window) {
#pragma unroll
        for (int j = 0; j < kAnyHPT; ++j) {
            const int g = wave + 4 * j;
            if (g < G) scores[(size_t)(kvh * G + g) * capacity + p0 + lane] = acc[j] * scale;
        }
    }
}

// rope_1d_batched (ops.rs:185-208) over n_heads contiguous heads of one
// vector in place: head blockIdx.x, pair i = threadIdx.x (head_dim / 2
// threads), angles as RopeArgs says.
__global__ __launch_bounds__(512) void rope_heads_kernel(float *__restrict__ vec, int pos, int head_dim, RopeArgs rope)
{
    const int half = head_dim >> 1, i = threadIdx.x;
    float c, sn;
    rope_cs(rope, pos, i, head_dim, c, sn);
    float *v = vec + (size_t)blockIdx.x * head_dim;
    const float v0 = v[i], v1 = v[i + half];
    v[i] = v0 * c - v1 * sn;
    v[i + half] = v0 * sn + v1 * c;
}

// act[i] = silu(g[i]) * u[i] with silu(x) = x / (1 + expf(-x)) (ops.rs:116-130),
// expf the glibc-exact port, so each element rounds as the CPU path's does.
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                                          float *__restrict__ act, int n, int expf_fused)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float x = g[i];
        act[i] = x / (1.0f + mrml_libm::expf(-x, expf_fused != 0)) * u[i];
    }
}

// out[i] = a[i] + b[i] (kernels.rs:732-744's rust_cuda_add_f32; one IEEE add).
__global__ __launch_bounds__(256) void add_rows_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                                       float *__restrict__ out, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

template <bool ROPE>
__global__ __launch_bounds__(kScoreT) void attn_scores2_kernel(const float *__restrict__ q_in,
                                                               uint16_t *__restrict__ k_cache,
                                                               uint16_t *__restrict__ v_cache,
                                                               const int32_t *__restrict__ d_pos, int n_past_arg,
                                                               int n_heads, int n_kv_heads, float scale, int capacity, int wlimit,
                                                               RopeArgs rope, float *__restrict__ scores, int q_stride)
{
    constexpr int HD = kAttnHD, P = kScoreP, half = HD / 2;
    __shared__ __align__(16) float q_s[4][HD];
    __shared__ __align__(16) uint8_t k_s[P * kKRow2];
    // query row blockIdx.z of a batch (prefill): rows q_stride floats apart
    // at consecutive positions, one score block per row
    q_in += (size_t)blockIdx.z * q_stride;
    scores += (size_t)blockIdx.z * n_heads * capacity;
    n_past_arg += (int)blockIdx.z;
    int window, start;
    attn_window(d_pos, n_past_arg, wlimit, window, start);
    const int p0 = blockIdx.x * P;
    const int kvh = blockIdx.y, G = n_heads / n_kv_heads, tid = threadIdx.x;
    const size_t kv_dim = (size_t)n_kv_heads * HD;
    const int pos = start + window - 1;  // the newest position
    const int rnew = window - 1 - p0;    // its row in this tile (valid when 0 <= rnew < P)
    const bool has_new = ROPE && rnew < P;
    // The newest position's rotated k and its v go to the caches from the
    // first workgroup past the window when the grid has one (it would exit
    // at once otherwise); the tile holding that position then only forms the
    // rotated row in LDS.  Stores in the tile's workgroup held its chain back
    // (its scores landed up to 1.5 us after the other tiles').
    const int ntile = (window + P - 1) / P;
    const bool spare = ntile < (int)gridDim.x;
    if (p0 >= window) {
        if (ROPE && (int)blockIdx.x == ntile && tid < half) {
            float c, sn;
            rope_cs(rope, pos, tid, HD, c, sn);
            const size_t crow = cache_row_of(pos, capacity) * kv_dim + (size_t)kvh * HD;
            const float *kh = q_in + (size_t)(n_heads + kvh) * HD;
            const float *vh = q_in + (size_t)(n_heads + n_kv_heads + kvh) * HD;
            const float k0 = kh[tid], k1 = kh[tid + half], v0 = vh[tid], v1 = vh[tid + half];
            k_cache[crow + tid] = f32_to_f16_rne(k0 * c - k1 * sn);
            k_cache[crow + tid + half] = f32_to_f16_rne(k0 * sn + k1 * c);
            v_cache[crow + tid] = f32_to_f16_rne(v0);
            v_cache[crow + tid + half] = f32_to_f16_rne(v1);
        }
        return;
    }
    // K tile: 2048 chunks of 16 B, chunk c of row r = c >> 5 at r*528 + (c & 31)*16
    constexpr int kChunks = P * (HD * 2 / 16), kPer = kChunks / kScoreT;
    u32x4 tmp[kPer];  // a native vector: arrays of HIP's uint4 struct end up in scratch memory
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = k * kScoreT + tid, r = c >> 5;
        const int pr = p0 + r < window ? p0 + r : window - 1;
        tmp[k] = reinterpret_cast<const u32x4 *>(k_cache + cache_row_of(start + pr, capacity) * kv_dim +
                                                 (size_t)kvh * HD)[c & 31];
    }
    // rotated (or copied) q of the group's heads: thread -> pairs (g, i)
    // with i = tid % 128 for every g, so one cos/sin per thread serves q and k
    static_assert(kScoreT % half == 0, "one rotation pair index per thread");
    float c = 1.0f, sn = 0.0f;
    if (ROPE) rope_cs(rope, pos, tid % half, HD, c, sn);
    for (int gi = tid; gi < G * half; gi += kScoreT) {
        const int g = gi / half, i = gi % half;
        const float *qh = q_in + (size_t)(kvh * G + g) * HD;
        const float v0 = qh[i], v1 = qh[i + half];
        if (ROPE) {
            q_s[g][i] = v0 * c - v1 * sn;
            q_s[g][i + half] = v0 * sn + v1 * c;
        } else {
            q_s[g][i] = v0;
            q_s[g][i + half] = v1;
        }
    }
    if (has_new) {
        const size_t crow = cache_row_of(pos, capacity) * kv_dim + (size_t)kvh * HD;
        uint16_t *krow = reinterpret_cast<uint16_t *>(k_s + rnew * kKRow2);
        if (tid < half) {
            const int i = tid;
            const float *kh = q_in + (size_t)(n_heads + kvh) * HD;
            const float v0 = kh[i], v1 = kh[i + half];
            const uint16_t k0 = f32_to_f16_rne(v0 * c - v1 * sn), k1 = f32_to_f16_rne(v0 * sn + v1 * c);
            krow[i] = k0;
            krow[i + half] = k1;
            if (!spare) {
                k_cache[crow + i] = k0;
                k_cache[crow + i + half] = k1;
            }
        } else if (!spare) {
            const int i = tid - half;
            const float *vh = q_in + (size_t)(n_heads + n_kv_heads + kvh) * HD;
            v_cache[crow + i] = f32_to_f16_rne(vh[i]);
            v_cache[crow + i + half] = f32_to_f16_rne(vh[i + half]);
        }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = k * kScoreT + tid, r = c >> 5;
        if (!(has_new && r == rnew)) *reinterpret_cast<u32x4 *>(k_s + r * kKRow2 + (c & 31) * 16) = tmp[k];
    }
    __syncthreads();
    const int g = tid >> 6, p = tid & 63;
    if (g >= G) return;
    const u32x4 *krow = reinterpret_cast<const u32x4 *>(k_s + p * kKRow2);
    const float4 *qg = reinterpret_cast<const float4 *>(q_s[g]);
    // -0.0 hidden from constant folding (an fma with a literal -0.0 addend
    // becomes a plain multiply), so q * f16 k maps to one v_fma_mix_f32
    float nz;
    asm volatile("v_mov_b32 %0, 0x80000000" : "=v"(nz));
    // 32 dims per step; the next step's K and q reads are issued before
    // this step's 32 dependent adds (double-buffered registers), so the
    // chain does not stop for an LDS round trip at every step
    float dot = -0.0f;
    constexpr int kSteps = HD / 32;
    u32x4 kw[2][4];
    float4 qa[2][8];
    auto fetch = [&](int st, int b) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            kw[b][u] = krow[4 * st + u];
            qa[b][2 * u] = qg[2 * (4 * st + u)];
            qa[b][2 * u + 1] = qg[2 * (4 * st + u) + 1];
        }
    };
    fetch(0, 0);
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const int b = st & 1;
        if (st + 1 < kSteps) fetch(st + 1, b ^ 1);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const u32x4 wv = kw[b][u];
            const uint32_t w[4] = {wv.x, wv.y, wv.z, wv.w};
            const float qv[8] = {qa[b][2 * u].x, qa[b][2 * u].y, qa[b][2 * u].z, qa[b][2 * u].w,
                                 qa[b][2 * u + 1].x, qa[b][2 * u + 1].y, qa[b][2 * u + 1].z, qa[b][2 * u + 1].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 kh = __builtin_bit_cast(_Float16, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
                dot = dot + __builtin_fmaf(qv[e], (float)kh, nz);
            }
        }
    }
    if (p0 + p < window) scores[(size_t)(kvh * G + g) * capacity + p0 + p] = dot * scale;
}

// Prefill form of the scores: positions tiled absolutely, so one K tile
// serves several query rows.  Workgroup (tile of 64 positions T0.., kv head,
// block of RB = 8 / G consecutive query rows): the tile's K rows are staged
// in LDS once, then wave w runs row w / G, head w % G of the group, lane p
// the chain of position T0 + p when the row's window holds it (the same
// arithmetic as attn_scores2_kernel: q . k from -0.0 in dim order, one
// product and one add per dim, times scale), stored at the position's index
// in that row's window.  Row z's position is n_past0 + z; t_lo is row 0's
// window start.
constexpr int kSRowsW = 8;  // waves per workgroup
template <int G>
__global__ __launch_bounds__(64 * kSRowsW) void attn_scores_rows_kernel(const float *__restrict__ q_in, int q_stride,
                                                                      const uint16_t *__restrict__ k_cache,
                                                                      int n_past0, int rows, int n_heads,
                                                                      int n_kv_heads, float scale, int capacity,
                                                                      int wlimit, int t_lo, float *__restrict__ scores)
{
    constexpr int HD = kAttnHD, P = kScoreP, RB = kSRowsW / G, NT = 64 * kSRowsW;
    __shared__ __align__(16) float q_s[RB * G][HD];
    __shared__ __align__(16) uint8_t k_s[P * kKRow2];
    // row blocks in reverse order: the latest rows, with the most tiles, are
    // dispatched first, so the launch does not end on them
    const int T0 = t_lo + (int)blockIdx.x * P, kvh = blockIdx.y, tid = threadIdx.x;
    const int z0 = ((int)gridDim.z - 1 - (int)blockIdx.z) * RB;
    const int zl = (z0 + RB < rows ? z0 + RB : rows) - 1;  // the block's last row
    int win0, start0, winl, startl;
    attn_window(nullptr, n_past0 + z0, wlimit, win0, start0);
    attn_window(nullptr, n_past0 + zl, wlimit, winl, startl);
    const int pos_l = n_past0 + zl;
    if (T0 > pos_l || T0 + P - 1 < start0) return;  // no row of the block has a position in this tile
    const size_t kv_dim = (size_t)n_kv_heads * HD;
    // K tile: 2048 chunks of 16 B (positions past the block's newest one
    // reload that row; their scores are not stored)
    constexpr int kChunks = P * (HD * 2 / 16), kPer = kChunks / NT;
    u32x4 tmp[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = k * NT + tid, r = c >> 5;
        const int t = T0 + r <= pos_l ? T0 + r : pos_l;
        tmp[k] = reinterpret_cast<const u32x4 *>(k_cache + cache_row_of(t, capacity) * kv_dim + (size_t)kvh * HD)[c & 31];
    }
    // q of the block's rows and the group's heads: RB*G*HD floats, float4 each
    for (int i = tid; i < RB * G * HD / 4; i += NT) {
        const int w = i / (HD / 4), e = i % (HD / 4), r = w / G, g = w % G;
        const int z = z0 + r < rows ? z0 + r : rows - 1;
        reinterpret_cast<float4 *>(q_s[w])[e] =
            reinterpret_cast<const float4 *>(q_in + (size_t)z * q_stride + (size_t)(kvh * G + g) * HD)[e];
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = k * NT + tid, r = c >> 5;
        *reinterpret_cast<u32x4 *>(k_s + r * kKRow2 + (c & 31) * 16) = tmp[k];
    }
    __syncthreads();
    const int w = tid >> 6, p = tid & 63;
    if (w >= RB * G) return;
    const int r = w / G, g = w % G, z = z0 + r, t = T0 + p;
    if (z >= rows) return;
    int window, start;
    attn_window(nullptr, n_past0 + z, wlimit, window, start);
    const u32x4 *krow = reinterpret_cast<const u32x4 *>(k_s + p * kKRow2);
    const float4 *qg = reinterpret_cast<const float4 *>(q_s[w]);
    float nz;
    asm volatile("v_mov_b32 %0, 0x80000000" : "=v"(nz));
    float dot = -0.0f;
    constexpr int kSteps = HD / 32;
    u32x4 kw[2][4];
    float4 qa[2][8];
    auto fetch = [&](int st, int b) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            kw[b][u] = krow[4 * st + u];
            qa[b][2 * u] = qg[2 * (4 * st + u)];
            qa[b][2 * u + 1] = qg[2 * (4 * st + u) + 1];
        }
    };
    fetch(0, 0);
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const int b = st & 1;
        if (st + 1 < kSteps) fetch(st + 1, b ^ 1);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const u32x4 wv = kw[b][u];
            const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
            const float qv[8] = {qa[b][2 * u].x, qa[b][2 * u].y, qa[b][2 * u].z, qa[b][2 * u].w,
                                 qa[b][2 * u + 1].x, qa[b][2 * u + 1].y, qa[b][2 * u + 1].z, qa[b][2 * u + 1].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 kh = __builtin_bit_cast(_Float16, (uint16_t)(wd[e >> 1] >> (16 * (e & 1))));
                dot = dot + __builtin_fmaf(qv[e], (float)kh, nz);
            }
        }
    }
    if (t >= start && t < start + window)
        scores[((size_t)z * n_heads + kvh * G + g) * capacity + (t - start)] = dot * scale;
}

// Softmax and weighted values, query head h, dims [32*ds, 32*ds + 32) per
// workgroup (blockIdx = (h, ds)):  max over the window; e_p = expf(score_p -
// max); sum = 0 + e_0 + e_1 + ... in order; p_p = e_p * (1/sum); out[d] = 0 +
// p_0 v_0[d] + p_1 v_1[d] + ... in order.  (The eight workgroups of a head
// each repeat the softmax; the weighted sum is bound by the CU's LDS
// bandwidth, so a narrower slice per workgroup runs it faster.)
//
// The weighted sum splits into independent products and one ordered chain of
// adds per dim.  Six producer waves stream V in tiles of kSVT positions
// (tiles in flight in registers, the first ones loaded before the softmax
// starts), form the products p_t * v_t[d] and store them to LDS as [d][t]
// (thread: 2 positions x 4 dims, one 8-byte store per dim); wave 0 runs the
// 32 chains (lanes 32..63 repeat lanes 0..31), lane d adding row d four
// positions per 16-byte read, one tile behind the producers (one barrier per
// tile, products double-buffered).
// Writes out (nullable) and the Q8_0 pack of the n_heads*head_dim output
// (nullable).  Dynamic LDS: capacity floats plus 4 (sv_lds).
constexpr int kSVD = 32;  // dims per workgroup
constexpr int kSVW = 8;   // waves: wave 0 adds; waves 1-3 and 5-7 produce; wave 4, which shares wave 0's SIMD, idles
constexpr int kSVT = 96;  // positions per tile: 48 position pairs x 8 dim quads = one per producer thread
constexpr int kSVS = kSVT + 12;  // product row stride (floats), 27 16-byte segments: measured on gfx950, 16-byte
                                 // reads of 64 rows at this stride run 1.4x faster than at 25 and 7.5x faster
                                 // than at 24 segments (bank conflicts)


// Producer thread pt (0..383) of tile t: positions 2*(pt >> 3) .. +1 of the
// tile, dims 4*(pt & 7) .. +3 of the slice; rows past the window reload the
// last row (their products are zeroed).  ring0 = cache row of the tile's
// first position (the window's rows are consecutive modulo capacity).  The
// slice's 32 dims are one block of a quantised cache row, so per position:
//   VF 0 (f16):  r = the four halves (8 bytes);
//   VF 1 (Q8_0): r.x = quants 4dq..4dq+3, r.y = the block's f16 scale;
//   VF 2 (Q4_0): r.x = bytes 4(dq&3)..+3 (dims 4dq.. are their low nibbles
//                for dq < 4, high nibbles after), r.y = the f16 scale.
// Quantised blocks are 2-byte aligned (34 and 18 bytes), read as halfwords.
constexpr int kSVPT = 64 * (kSVW - 2);  // producer threads
constexpr int kSVR = 2;                 // positions per producer thread
static_assert(kSVT / kSVR * (kSVD / 4) == kSVPT, "one position pair x dim quad per producer thread");
template <int VF>
__device__ __forceinline__ void sv_tile_load(u32x2 (&r)[kSVR], const uint8_t *vslice, int t, int window, int ring0,
                                             int capacity, size_t row_bytes, int pt)
{
    const int tq = pt >> 3, dq = pt & 7;
#pragma unroll
    for (int i = 0; i < kSVR; ++i) {
        int rr = kSVR * tq + i;
        rr = t * kSVT + rr < window ? rr : window - 1 - t * kSVT;
        int row = ring0 + rr;
        row = row >= capacity ? row - capacity : row;
        const uint8_t *blk = vslice + (size_t)row * row_bytes;
        if constexpr (VF == 0) {
            r[i] = reinterpret_cast<const u32x2 *>(blk)[dq];
        } else {
            const uint16_t *h = reinterpret_cast<const uint16_t *>(blk);
            const int w = 1 + 2 * (VF == 1 ? dq : (dq & 3));  // halfword of byte 2 + 4*(dq or dq & 3)
            r[i].x = (uint32_t)h[w] | ((uint32_t)h[w + 1] << 16);
            r[i].y = h[0];
        }
    }
}

// Softmax weights of the producer's two positions: from the normalised
// window in LDS, or (LONG, windows too long for LDS) formed again from the
// global scores exactly as the LDS form forms them, expf(s - max) times
// 1/sum when sum > 0.  Positions past the window take a clamped in-window
// score (their products are zeroed).
struct SvWeights {
    const float *sc;  // the head's scores (LONG)
    float mx, inv;
    bool scaled, fused_exp;
    const uint64_t *exp_tab;
};

template <bool LONG, int VF>
__device__ __forceinline__ void sv_products(const u32x2 (&r)[kSVR], const float *e_s, const SvWeights &sw,
                                            float (*prod)[kSVS], int t, int window, int pt)
{
    const int tq = pt >> 3, dq = pt & 7, pos0 = t * kSVT + kSVR * tq;
    float w4[kSVR];
    if (LONG) {
#pragma unroll
        for (int i = 0; i < kSVR; ++i) {
            const int p = pos0 + i < window ? pos0 + i : window - 1;
            const float e = mrml_libm::expf_t(sw.sc[p] - sw.mx, sw.fused_exp, sw.exp_tab);
            w4[i] = sw.scaled ? e * sw.inv : e;
        }
    } else {
        const float2 pw = reinterpret_cast<const float2 *>(e_s)[(pos0 < window ? pos0 : 0) >> 1];
        w4[0] = pw.x;
        w4[1] = pw.y;
    }
    float pv[4][kSVR];  // [dim][position]
#pragma unroll
    for (int i = 0; i < kSVR; ++i) {
        const bool live = pos0 + i < window;
        if constexpr (VF == 0) {
            const uint32_t lo = r[i].x, hi = r[i].y;
            const float v[4] = {f16_bits_to_f32(lo & 0xffffu), f16_bits_to_f32(lo >> 16),
                                f16_bits_to_f32(hi & 0xffffu), f16_bits_to_f32(hi >> 16)};
#pragma unroll
            for (int d = 0; d < 4; ++d) pv[d][i] = live ? w4[i] * v[d] : 0.0f;
        } else {
            // KvCacheRow::add_head_scaled (kv_cache.rs:97-125): dd = d * p,
            // then dd * q per value, each product rounded
            const float dd = f16_bits_to_f32(r[i].y) * w4[i];
            const int sh = (VF == 2 && dq >= 4) ? 4 : 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t b = (r[i].x >> (8 * d)) & 0xffu;
                const int qv = VF == 1 ? (int)(int8_t)b : (int)((b >> sh) & 15u) - 8;
                pv[d][i] = live ? dd * (float)qv : 0.0f;
            }
        }
    }
#pragma unroll
    for (int d = 0; d < 4; ++d)
        *reinterpret_cast<float2 *>(&prod[4 * dq + d][kSVR * tq]) = make_float2(pv[d][0], pv[d][1]);
}

// LONG (capacities past kSVShortCap): the window's weights do not fit in
// LDS.  The sum then runs over chunks of kSVChunk - 1 exps staged in LDS,
// each chunk's exact sequential sum started from the running sum (prepended
// as the chunk's first term: s = 0 + s_prev is exact, so the chunked sums
// equal the one sequential loop), and the producers form their weights from
// the global scores.  Dynamic LDS: kSVChunk floats, kSVChunk flag bytes and
// the block sum's Shared.
constexpr int kSVShortCap = 6144;  // the LDS form keeps capacity floats of weights
constexpr int kSVChunk = 8192;     // LONG: terms per exact block sum (16 per thread)
static_assert(kSVChunk <= mrml_xsum::kMaxPerThread * 64 * kSVW, "one block sum per chunk");

__host__ __device__ constexpr bool sv_long(int capacity) { return capacity > kSVShortCap; }
inline size_t sv_lds(int capacity)
{
    return sv_long(capacity) ? (size_t)kSVChunk * 5 + sizeof(mrml_xsum::Shared) : (size_t)capacity * sizeof(float) + 16;
}

// VF: the V cache's format (0 f16, 1 Q8_0, 2 Q4_0; KvCacheFormat::cuda_code);
// grid (n_heads, head_dim / 32, rows).
template <bool LONG, int VF>
__global__ __launch_bounds__(64 * kSVW) void attn_softmax_v_kernel(const float *__restrict__ scores,
                                                             const uint8_t *__restrict__ v_cache,
                                                             const int32_t *__restrict__ d_pos, int n_past_arg,
                                                             int n_heads, int n_kv_heads, int head_dim, int capacity,
                                                             int wlimit, int expf_fused, float *__restrict__ out,
                                                             uint8_t *__restrict__ pack)
{
    const int HD = head_dim;
    extern __shared__ __align__(16) float e_s[];
    __shared__ float red[kSVW];
    __shared__ __align__(16) float prod[2][kSVD][kSVS];
    __shared__ __align__(16) mrml_xsum::Shared4 sum_xs[1];
    __shared__ uint64_t exp_tab[32];
    mrml_xsum::Shared4 *sum_x = sum_xs;
    scores += (size_t)blockIdx.z * n_heads * capacity;  // query row blockIdx.z of a batch (prefill; no pack)
    if (out) out += (size_t)blockIdx.z * n_heads * HD;
    n_past_arg += (int)blockIdx.z;
    int window, start;
    attn_window(d_pos, n_past_arg, wlimit, window, start);
    const int h = blockIdx.x, ds = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int G = n_heads / n_kv_heads, kvh = h / G;
    const float *sc = scores + (size_t)h * capacity;
    // bytes of one cached 32-value block, of a cache row, and the slice's offset
    constexpr size_t kBB = VF == 0 ? 64 : (VF == 1 ? 34 : 18);
    const size_t kv_dim = (size_t)n_kv_heads * (HD / kSVD) * kBB;
    const uint8_t *vslice = v_cache + ((size_t)kvh * (HD / kSVD) + ds) * kBB;
    const int ntiles = (window + kSVT - 1) / kSVT;
    const bool producer = (wave & 3) != 0;
    const int pt = (wave < 4 ? wave - 1 : wave - 2) * 64 + lane;
    // cache row of tile t's first position: ring row of `start`, advanced by kSVT per tile
    const int ring_start = (int)cache_row_of(start, capacity), step = kSVT % (capacity > 0 ? capacity : 1 << 30);
    auto ring_next = [&](int r) { return r + step >= capacity ? r + step - capacity : r + step; };
    // tiles t .. t+3 in flight in registers (slot t % 4); ring[k] = cache row of the slot's tile
    u32x2 vt[4][kSVR];
    int ring[4];
    ring[0] = ring_start;
#pragma unroll
    for (int k = 1; k < 4; ++k) ring[k] = ring_next(ring[k - 1]);
    if (producer) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (k < ntiles) sv_tile_load<VF>(vt[k], vslice, k, window, ring[k], capacity, kv_dim, pt);
    }

    if (tid < 32) exp_tab[tid] = mrml_libm::kExpfT.t[tid];  // read before the max's barrier
    // max over the window (exact in any order): DPP within each half-wave.
    // Thread t takes positions 4t..4t+3 (+2048 per pass), so up to 2048
    // positions its exps stay in registers for the sum.
    constexpr int kSVE = 4 * 64 * kSVW;  // positions per pass
    const float4 *sc4 = reinterpret_cast<const float4 *>(sc);
    const bool sc_a16 = (reinterpret_cast<uintptr_t>(sc) & 15) == 0;  // a capacity not a multiple of 4: scalar loads
    float4 sv = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    float mx = -INFINITY;
    for (int p0 = 0; p0 < window; p0 += kSVE) {
        const int p = p0 + 4 * tid;
        float4 v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (sc_a16 && p + 3 < window) {
            v = sc4[p >> 2];
        } else if (p < window) {
            v.x = sc[p];
            if (p + 1 < window) v.y = sc[p + 1];
            if (p + 2 < window) v.z = sc[p + 2];
            if (p + 3 < window) v.w = sc[p + 3];
        }
        if (p0 == 0) sv = v;
        mx = fmaxf(mx, fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
    }
    mx = max32(mx);
    mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx), 32)));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kSVW; ++w) mx = fmaxf(mx, red[w]);
    const bool fused_exp = expf_fused != 0;
    float sum;
    if (window <= kSVE) {
        // exps in registers; the ordered sum over the block (exact_sum.h)
        const int p = 4 * tid;
        float4 e = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (p < window) e.x = mrml_libm::expf_t(sv.x - mx, fused_exp, exp_tab);
        if (p + 1 < window) e.y = mrml_libm::expf_t(sv.y - mx, fused_exp, exp_tab);
        if (p + 2 < window) e.z = mrml_libm::expf_t(sv.z - mx, fused_exp, exp_tab);
        if (p + 3 < window) e.w = mrml_libm::expf_t(sv.w - mx, fused_exp, exp_tab);
        if (LONG) {
        } else if (p + 3 < window) {
            reinterpret_cast<float4 *>(e_s)[tid] = e;
        } else if (p < window) {
            e_s[p] = e.x;
            if (p + 1 < window) e_s[p + 1] = e.y;
            if (p + 2 < window) e_s[p + 2] = e.z;
        }
        sum = mrml_xsum::block_seq_sum_nonneg4(e, window, *sum_x);
    } else if (LONG) {
        uint8_t *flags = reinterpret_cast<uint8_t *>(e_s + kSVChunk);
        mrml_xsum::Shared &xs = *reinterpret_cast<mrml_xsum::Shared *>(flags + kSVChunk);
        float s = 0.0f;
        for (int c0 = 0; c0 < window; c0 += kSVChunk - 1) {
            const int n = window - c0 < kSVChunk - 1 ? window - c0 : kSVChunk - 1;
            if (tid == 0) e_s[0] = s;
            for (int i = tid; i < n; i += 64 * kSVW) e_s[1 + i] = mrml_libm::expf_t(sc[c0 + i] - mx, fused_exp, exp_tab);
            __syncthreads();
            s = mrml_xsum::block_seq_sum_nonneg(e_s, n + 1, flags, xs);  // ends with a barrier
        }
        sum = s;
    } else {
        for (int p = tid; p < window; p += 64 * kSVW) e_s[p] = mrml_libm::expf_t(sc[p] - mx, fused_exp, exp_tab);
        __syncthreads();
        float *bcast = e_s + capacity;
        if (wave == 0) {
            const float s0 = seq_sum(e_s, window);
            if (lane == 0) *bcast = s0;
        }
        __syncthreads();
        sum = *bcast;
    }
    const SvWeights sw{sc, mx, sum > 0.0f ? 1.0f / sum : 1.0f, sum > 0.0f, fused_exp, exp_tab};
    if (!LONG && sum > 0.0f) {
        for (int p = tid; p < window; p += 64 * kSVW) e_s[p] = e_s[p] * sw.inv;
    }
    __syncthreads();

    float acc = 0.0f;
    // Row `lane` of the tile: all 24 16-byte reads are issued before the
    // first add (pinned by the scheduling barrier: under the producers' LDS
    // traffic a read takes a few hundred cycles, more than a short prefetch
    // covers), then the 96 ordered adds.  Zeroed tail products leave acc
    // unchanged (it never holds -0).
    auto chain = [&](int t) {
        const float4 *row = reinterpret_cast<const float4 *>(prod[t & 1][lane & (kSVD - 1)]);
        float4 b[kSVT / 4];
#pragma unroll
        for (int i = 0; i < kSVT / 4; ++i) b[i] = row[i];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < kSVT / 4; ++i) {
            acc = acc + b[i].x;
            acc = acc + b[i].y;
            acc = acc + b[i].z;
            acc = acc + b[i].w;
        }
    };
    // buffer (t+1)&1 was last read by wave 0 in tile t-1, before barrier t
    auto tile = [&](int t, int k) {  // k = t % 4, a compile-time slot
        if (producer) {
            sv_products<LONG, VF>(vt[k], e_s, sw, prod[t & 1], t, window, pt);
            if (t + 4 < ntiles) {
                ring[k] = ring_next(ring_next(ring_next(ring_next(ring[k]))));
                sv_tile_load<VF>(vt[k], vslice, t + 4, window, ring[k], capacity, kv_dim, pt);
            }
        }
        __syncthreads();
        if (wave == 0 && lane < kSVD) chain(t);
    };
    for (int t = 0; t < ntiles; t += 4) {
        tile(t, 0);
        if (t + 1 < ntiles) tile(t + 1, 1);
        if (t + 2 < ntiles) tile(t + 2, 2);
        if (t + 3 < ntiles) tile(t + 3, 3);
    }

    if (wave == 0) {
        const int o = h * HD + ds * kSVD + (lane & (kSVD - 1));
        if (out && lane < kSVD) out[o] = acc;
        if (pack) {
            uint32_t dbits;
            int s;
            const int qv = q8_0_block32(acc, dbits, s);
            const int nb = n_heads * HD / 32, blk = o >> 5;
            if (lane < kSVD) pack[o] = (uint8_t)(int8_t)qv;
            if (lane == 0) {
                reinterpret_cast<float *>(pack + (size_t)nb * 32)[blk] = f16_bits_to_f32(dbits);
                reinterpret_cast<int32_t *>(pack + (size_t)nb * 36)[blk] = s;
            }
        }
    }
}

// ---- split-K decode attention: the decode step's tolerance path ---------------
// The same attention (model.rs:1457-1590, softmax ops.rs:133-158) evaluated in
// parallel over the window instead of in the reference's sequential order,
// as flash decoding does: the window (the last min(n_past+1, capacity)
// positions, oldest first) is cut into tiles of kSplitP positions and
// workgroup (tile, kv head) forms, for each query head of the group,
//   m = max_p s_p,  l = sum_p e_p,  o[d] = sum_p e_p v_p[d],
//   s_p = scale * (q . k_p),  e_p = expf(s_p - m),
// over its tile (f32, fixed-order tree sums: deterministic); then
// attn_combine_kernel merges the tiles of a head,
//   M = max_t m_t,  L = sum_t l_t expf(m_t - M),  out[d] = (sum_t o_t[d] expf(m_t - M)) / L,
// in tile order and writes the Q8_0 pack of the output for the next product.
// Results are within a few ulps of the sequential ones (the tests bound them
// at 1e-5 relative to the output's largest magnitude), not bit-identical.
//
// With ROPE, q comes raw from the stacked q|k|v vector and is rotated here
// (cos/sin from the host table when pos < n_table), and the workgroup whose
// tile holds the newest position rotates that position's k, rounds k and v
// to f16 (RNE, as the cache stores them), uses them for that row and appends
// them to the caches -- what attn_scores2_kernel<true> does for the exact
// path.  Workgroups of tiles past the window exit at once.
constexpr int kSplitP = 32;                    // positions per tile (two lanes each: dims 0..127, 128..255)
constexpr int kSplitT = 256;                   // threads per workgroup
constexpr int kSplitKRow = kAttnHD * 2 + 16;   // padded K row in LDS, bytes (conflict-free 16-byte reads of 64 rows)
constexpr int kSplitPart = kAttnHD + 4;        // floats per partial: o[256], m, l, pad

__device__ __forceinline__ float wave_max_f32(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

template <bool ROPE>
__global__ __launch_bounds__(kSplitT) void attn_split_kernel(const float *__restrict__ q_in,
                                                             uint16_t *__restrict__ k_cache,
                                                             uint16_t *__restrict__ v_cache,
                                                             const int32_t *__restrict__ d_pos, int n_past_arg,
                                                             int n_heads, int n_kv_heads, float scale, int capacity, int wlimit,
                                                             RopeArgs rope, float *__restrict__ part, int max_tiles)
{
    constexpr int HD = kAttnHD, P = kSplitP, half = HD / 2;
    __shared__ __align__(16) float q_s[8][HD];
    __shared__ __align__(16) uint8_t k_s[P * kSplitKRow];
    __shared__ __align__(16) uint16_t v_s[P][HD];
    __shared__ __align__(16) float e_s[8][P];
    static_assert(P == 32, "two lanes per position");
    int window, start;
    attn_window(d_pos, n_past_arg, wlimit, window, start);
    const int tile = blockIdx.x, p0 = tile * P;
    if (p0 >= window) return;
    const int kvh = blockIdx.y, G = n_heads / n_kv_heads, tid = threadIdx.x;
    const size_t kv_dim = (size_t)n_kv_heads * HD;
    const int pos = start + window - 1;  // the newest position
    const int rnew = window - 1 - p0;    // its row in this tile (valid when < P)
    const bool has_new = ROPE && rnew < P;
    // K and V tiles: P*32 chunks of 16 B each, chunk c of row r = c >> 5;
    // rows past the window reload the last row (their scores are masked)
    constexpr int kChunks = P * (HD * 2 / 16), kPer = kChunks / kSplitT;
    u32x4 kt[kPer], vt[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = k * kSplitT + tid, r = c >> 5;
        const int pr = p0 + r < window ? p0 + r : window - 1;
        const size_t off = cache_row_of(start + pr, capacity) * kv_dim + (size_t)kvh * HD;
        kt[k] = reinterpret_cast<const u32x4 *>(k_cache + off)[c & 31];
        vt[k] = reinterpret_cast<const u32x4 *>(v_cache + off)[c & 31];
    }
    // q of the group's heads, rotated with ROPE (thread -> pair i = tid % half)
    static_assert(kSplitT % half == 0, "one rotation pair index per thread");
    float c = 1.0f, sn = 0.0f;
    if (ROPE) rope_cs(rope, pos, tid % half, HD, c, sn);
    for (int gi = tid; gi < G * half; gi += kSplitT) {
        const int g = gi / half, i = gi % half;
        const float *qh = q_in + (size_t)(kvh * G + g) * HD;
        const float v0 = qh[i], v1 = qh[i + half];
        q_s[g][i] = ROPE ? v0 * c - v1 * sn : v0;
        q_s[g][i + half] = ROPE ? v0 * sn + v1 * c : v1;
    }
    if (has_new) {
        const size_t crow = cache_row_of(pos, capacity) * kv_dim + (size_t)kvh * HD;
        if (tid < half) {
            const int i = tid;
            const float *kh = q_in + (size_t)(n_heads + kvh) * HD;
            const float v0 = kh[i], v1 = kh[i + half];
            const uint16_t k0 = f32_to_f16_rne(v0 * c - v1 * sn), k1 = f32_to_f16_rne(v0 * sn + v1 * c);
            uint16_t *krow = reinterpret_cast<uint16_t *>(k_s + rnew * kSplitKRow);
            krow[i] = k0;
            krow[i + half] = k1;
            k_cache[crow + i] = k0;
            k_cache[crow + i + half] = k1;
        } else {
            const int i = tid - half;
            const float *vh = q_in + (size_t)(n_heads + n_kv_heads + kvh) * HD;
            const uint16_t w0 = f32_to_f16_rne(vh[i]), w1 = f32_to_f16_rne(vh[i + half]);
            v_s[rnew][i] = w0;
            v_s[rnew][i + half] = w1;
            v_cache[crow + i] = w0;
            v_cache[crow + i + half] = w1;
        }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int cc = k * kSplitT + tid, r = cc >> 5;
        if (!(has_new && r == rnew)) {
            *reinterpret_cast<u32x4 *>(k_s + r * kSplitKRow + (cc & 31) * 16) = kt[k];
            reinterpret_cast<u32x4 *>(&v_s[r][0])[cc & 31] = vt[k];
        }
    }
    __syncthreads();
    const int wave = tid >> 6, lane = tid & 63;
    const int ntile = window - p0 < P ? window - p0 : P;  // live rows of the tile (masked scores past it)
    const int pl = lane & (P - 1), dh = lane / P;  // position in the tile, half of the dims
    for (int g = wave; g < G; g += kSplitT / 64) {
        // score of position p0 + pl: lane pl sums dims 0..127 and lane pl + 32
        // dims 128..255, four partial dot products each
        const u32x4 *krow = reinterpret_cast<const u32x4 *>(k_s + pl * kSplitKRow) + dh * (HD / 16);
        const float4 *qg = reinterpret_cast<const float4 *>(q_s[g]) + dh * (HD / 8);
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int d8 = 0; d8 < HD / 16; ++d8) {
            const u32x4 kw = krow[d8];
            const float4 qa = qg[2 * d8], qb = qg[2 * d8 + 1];
            const uint32_t w[4] = {kw.x, kw.y, kw.z, kw.w};
            const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                a[e & 3] = __builtin_fmaf(qv[e], f16_bits_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xffffu), a[e & 3]);
        }
        const bool live = pl < ntile;
        const float part_dot = (a[0] + a[1]) + (a[2] + a[3]);
        const float sc = (part_dot + __shfl_xor(part_dot, 32, 64)) * scale;  // the same in both lanes
        const float m = wave_max_f32(live ? sc : -INFINITY);
        const float e = live ? __builtin_expf(sc - m) : 0.0f;
        const float l = mrml_xsum::wave_sum_f32(dh == 0 ? e : 0.0f);
        if (dh == 0) e_s[g][pl] = e;
        __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS writes done (lgkmcnt 0)
        __builtin_amdgcn_wave_barrier();     // (LDS accesses of one wave run in order)
        // o[d] for d = 4*lane .. 4*lane+3 over all P rows of the tile (rows
        // past the window have e = 0 and finite values), eight rows per step
        // with their LDS reads issued together, even and odd rows in two
        // accumulators
        float4 oa = make_float4(0.0f, 0.0f, 0.0f, 0.0f), ob = oa;
        const float4 *e4 = reinterpret_cast<const float4 *>(e_s[g]);
#pragma unroll 2
        for (int p = 0; p < P; p += 8) {
            const float4 ea = e4[p / 4], eb = e4[p / 4 + 1];
            const float ep[8] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
            u32x2 vv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) vv[k] = reinterpret_cast<const u32x2 *>(&v_s[p + k][0])[lane];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                float4 &o = (k & 1) ? ob : oa;
                o.x = __builtin_fmaf(ep[k], f16_bits_to_f32(vv[k].x & 0xffffu), o.x);
                o.y = __builtin_fmaf(ep[k], f16_bits_to_f32(vv[k].x >> 16), o.y);
                o.z = __builtin_fmaf(ep[k], f16_bits_to_f32(vv[k].y & 0xffffu), o.z);
                o.w = __builtin_fmaf(ep[k], f16_bits_to_f32(vv[k].y >> 16), o.w);
            }
        }
        const float4 o = make_float4(oa.x + ob.x, oa.y + ob.y, oa.z + ob.z, oa.w + ob.w);
        float *pp = part + ((size_t)(kvh * G + g) * max_tiles + tile) * kSplitPart;
        reinterpret_cast<float4 *>(pp)[lane] = o;
        if (lane == 0) {
            pp[HD] = m;
            pp[HD + 1] = l;
        }
    }
}

// Prefill form of attn_softmax_v_kernel: one workgroup per (query row, kv
// head), thread d = output dim d of each of the group's G query heads.  Each
// row's arithmetic is the decode form's -- per head the max over the window,
// e_p = expf(s_p - max), the ordered exp sum, p_p = e_p * (1/sum), out[d] =
// 0 + p_0 v_0[d] + p_1 v_1[d] + ... in order -- but the softmax is formed
// once per head rather than once per 32-dim slice, and each thread runs its
// dim's chains, one per head of the group, over V rows read straight from
// the cache: every V load feeds G chains, and the next 32 positions' loads
// are in flight while the current 32 are added.  The decode form spreads
// one long row over eight workgroups to cut its latency; a prefill chunk has
// rows enough to fill the GPU this way.  Windows up to kRowsSvMax positions
// (one exact block sum per head) and groups of G <= kRowsSvG heads (a
// compile-time count, so the per-position work has no head loop or test).
// Dynamic LDS: the group's weights, G rows of `span` floats (the launch's
// widest window) at a stride of a multiple of 4 floats, then span flag bytes.
constexpr int kRowsSvMax = mrml_xsum::kMaxPerThread * kAttnHD;  // 4096
constexpr int kRowsSvG = 4;
constexpr int kRowsSvB = 32;  // positions per load batch
inline int rows_sv_stride(int span) { return (span + 3) & ~3; }
inline size_t rows_sv_lds(int g, int span)
{
    return (size_t)g * rows_sv_stride(span) * sizeof(float) + ((span + 15) & ~15);
}

// SHORT (windows up to 4 * kAttnHD): thread d takes positions 4d..4d+3, its
// exps stay in registers for the register form of the exact sum.
template <int G, bool SHORT>
__global__ __launch_bounds__(kAttnHD) void attn_softmax_v_rows_kernel(const float *__restrict__ scores,
                                                                      const uint16_t *__restrict__ v_cache,
                                                                      int n_past0, int n_heads, int n_kv_heads,
                                                                      int capacity, int wlimit, int expf_fused,
                                                                      float *__restrict__ out, int span)
{
    constexpr int HD = kAttnHD, B = kRowsSvB;
    extern __shared__ __align__(16) float e_dyn[];  // [G][span] weights, then span flag bytes
    __shared__ float red[HD / 64];
    __shared__ uint64_t exp_tab[32];
    // rows in reverse order: the longest windows are dispatched first, so the
    // launch does not end on them
    const int kvh = blockIdx.x, z = (int)gridDim.y - 1 - (int)blockIdx.y, d = threadIdx.x, stride = (span + 3) & ~3;
    uint8_t *flags = reinterpret_cast<uint8_t *>(e_dyn + (size_t)G * stride);
    auto e_s = [&](int g) { return e_dyn + (size_t)g * stride; };
    int window, start;
    attn_window(nullptr, n_past0 + z, wlimit, window, start);
    if (d < 32) exp_tab[d] = mrml_libm::kExpfT.t[d];
    const bool fused = expf_fused != 0;
    if constexpr (SHORT) {
        __shared__ mrml_xsum::Shared4 xs4;
        const int p = 4 * d;
#pragma unroll 1
        for (int g = 0; g < G; ++g) {
            const float *sc = scores + ((size_t)z * n_heads + kvh * G + g) * capacity;
            float sv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[i] = p + i < window ? sc[p + i] : -INFINITY;
            float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));  // the max is exact in any order
            mx = wave_max_f32(mx);
            if ((d & 63) == 0) red[d >> 6] = mx;
            __syncthreads();
            mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = p + i < window ? mrml_libm::expf_t(sv[i] - mx, fused, exp_tab) : 0.0f;
            // (its first barrier also orders every thread's read of red
            // before the next head rewrites it)
            const float sum = mrml_xsum::block_seq_sum_nonneg4(make_float4(e[0], e[1], e[2], e[3]), window, xs4);
            const float inv = sum > 0.0f ? 1.0f / sum : 1.0f;
            float *eg = e_s(g);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (p + i < window) eg[p + i] = sum > 0.0f ? e[i] * inv : e[i];
        }
    } else {
#pragma unroll 1
    for (int g = 0; g < G; ++g) {
        const float *sc = scores + ((size_t)z * n_heads + kvh * G + g) * capacity;
        float mx = -INFINITY;  // the max is exact in any order
        for (int p = d; p < window; p += HD) mx = fmaxf(mx, sc[p]);
        mx = wave_max_f32(mx);
        if ((d & 63) == 0) red[d >> 6] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        float *eg = e_s(g);
        for (int p = d; p < window; p += HD) eg[p] = mrml_libm::expf_t(sc[p] - mx, fused, exp_tab);
        __syncthreads();  // also: every thread has read red before the next head rewrites it
        __shared__ mrml_xsum::Shared xs;
        const float sum = mrml_xsum::block_seq_sum_nonneg(eg, window, flags, xs);  // ends with a barrier
        if (sum > 0.0f) {
            const float inv = 1.0f / sum;
            for (int p = d; p < window; p += HD) eg[p] = eg[p] * inv;
        }
    }
    }
    __syncthreads();
    const size_t kv_dim = (size_t)n_kv_heads * HD;
    const uint16_t *vb = v_cache + (size_t)kvh * HD + d;
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
    int row = (int)cache_row_of(start, capacity);  // the window's rows are consecutive modulo capacity
    // unconditional loads (row stays a cache row; positions past the window
    // are skipped by add), so all B of them are issued before any is used
    auto load = [&](float (&v)[B], int) {
        uint16_t raw[B];
#pragma unroll
        for (int k = 0; k < B; ++k) {
            raw[k] = vb[(size_t)row * kv_dim];
            row = row + 1 == capacity ? 0 : row + 1;
        }
#pragma unroll
        for (int k = 0; k < B; ++k) v[k] = f16_bits_to_f32(raw[k]);
    };
    // a batch inside the window: each head's weights read four positions at
    // a time (float4 broadcasts), no per-position test
    auto add_full = [&](const float (&v)[B], int t0) {
#pragma unroll
        for (int i = 0; i < B / 4; ++i) {
            float4 e4[G];
#pragma unroll
            for (int g = 0; g < G; ++g) e4[g] = reinterpret_cast<const float4 *>(e_s(g) + t0)[i];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                acc[g] = acc[g] + e4[g].x * v[4 * i];
                acc[g] = acc[g] + e4[g].y * v[4 * i + 1];
                acc[g] = acc[g] + e4[g].z * v[4 * i + 2];
                acc[g] = acc[g] + e4[g].w * v[4 * i + 3];
            }
        }
    };
    // the window's last, partial batch
    auto add_part = [&](const float (&v)[B], int t0) {
#pragma unroll
        for (int k = 0; k < B; ++k) {
            if (t0 + k < window) {
#pragma unroll
                for (int g = 0; g < G; ++g) acc[g] = acc[g] + e_s(g)[t0 + k] * v[k];
            }
        }
    };
    float va[B], vb2[B];
    load(va, 0);
    int t0 = 0;
    for (; t0 + 2 * B <= window; t0 += 2 * B) {
        load(vb2, t0 + B);  // in flight while va is added
        add_full(va, t0);
        load(va, t0 + 2 * B);
        add_full(vb2, t0 + B);
    }
    if (t0 + B <= window) {
        load(vb2, t0 + B);
        add_full(va, t0);
        add_part(vb2, t0 + B);
    } else {
        add_part(va, t0);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) out[((size_t)z * n_heads + kvh * G + g) * HD + d] = acc[g];
}

// Merges the tiles of head blockIdx.x (thread d = output dim d), in tile
// order, and writes out (nullable) and the Q8_0 pack (nullable) of the
// n_heads*256 output.
__global__ __launch_bounds__(kAttnHD) void attn_combine_kernel(const float *__restrict__ part,
                                                               const int32_t *__restrict__ d_pos, int n_past_arg,
                                                               int capacity, int wlimit, int max_tiles, int n_heads,
                                                               float *__restrict__ out, uint8_t *__restrict__ pack)
{
    constexpr int HD = kAttnHD, kMaxTiles = (kSVShortCap + kSplitP - 1) / kSplitP;
    __shared__ float m_s[kMaxTiles], w_s[kMaxTiles], l_s[kMaxTiles];
    __shared__ float red[HD / 64];
    static_assert(kMaxTiles <= HD, "one tile's (m, l) per thread");
    const int h = blockIdx.x, d = threadIdx.x, tl = max_tiles - 1;
    const float *ph = part + (size_t)h * max_tiles * kSplitPart;
    // The first kPre tiles' values and tile d's (m, l) are loaded before the
    // window is known, beside the position's load (indices clamped to the
    // buffer's tiles; tiles past the window are never used): one round trip
    // for windows up to kPre tiles.
    constexpr int kPre = 32;
    float pv[kPre];
#pragma unroll
    for (int k = 0; k < kPre; ++k) pv[k] = ph[(size_t)(k < tl ? k : tl) * kSplitPart + d];
    const size_t td = (size_t)(d < tl ? d : tl) * kSplitPart;
    const float m_d = ph[td + HD], l_d = ph[td + HD + 1];
    int window, start;
    attn_window(d_pos, n_past_arg, wlimit, window, start);
    const int ntiles = (window + kSplitP - 1) / kSplitP;
    float L = 0.0f, o = 0.0f;
    if (ntiles <= kMaxTiles) {
        if (d < ntiles) {
            m_s[d] = m_d;
            l_s[d] = l_d;
        }
        __syncthreads();
        float M = -INFINITY;
        for (int t = 0; t < ntiles; ++t) M = fmaxf(M, m_s[t]);
        for (int t = d; t < ntiles; t += HD) w_s[t] = __builtin_expf(m_s[t] - M);
        __syncthreads();
        // L and o in tile order (every thread forms the same L)
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            if (k < ntiles) {  // uniform
                L = L + l_s[k] * w_s[k];
                o = o + pv[k] * w_s[k];
            }
        }
        int t = kPre;
        for (; t + 8 <= ntiles; t += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = ph[(size_t)(t + k) * kSplitPart + d];  // eight loads in flight
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                L = L + l_s[t + k] * w_s[t + k];
                o = o + v[k] * w_s[t + k];
            }
        }
        for (; t < ntiles; ++t) {
            L = L + l_s[t] * w_s[t];
            o = o + ph[(size_t)t * kSplitPart + d] * w_s[t];
        }
    } else {
        // windows past the LDS arrays: the same values in the same order, each
        // tile's (m, l) read where it lies and its weight formed per thread
        float M = -INFINITY;
        for (int t = d; t < ntiles; t += HD) M = fmaxf(M, ph[(size_t)t * kSplitPart + HD]);
        M = wave_max_f32(M);
        if ((d & 63) == 0) red[d >> 6] = M;
        __syncthreads();
        M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        for (int t = 0; t < ntiles; t += 8) {
            float v[8], mt[8], lt[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const size_t at = (size_t)(t + k < ntiles ? t + k : t) * kSplitPart;
                v[k] = ph[at + d];
                mt[k] = ph[at + HD];
                lt[k] = ph[at + HD + 1];
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (t + k < ntiles) {
                    const float w = __builtin_expf(mt[k] - M);
                    L = L + lt[k] * w;
                    o = o + v[k] * w;
                }
            }
        }
    }
    const float v = o / L;
    const int idx = h * HD + d;
    if (out) out[idx] = v;
    if (pack) {
        uint32_t dbits;
        int qs;
        const int qv = q8_0_block32(v, dbits, qs);  // 32-lane blocks: block idx / 32
        const int nb = n_heads * HD / 32, blk = idx >> 5;
        pack[idx] = (uint8_t)(int8_t)qv;
        if ((idx & 31) == 0) {
            reinterpret_cast<float *>(pack + (size_t)nb * 32)[blk] = f16_bits_to_f32(dbits);
            reinterpret_cast<int32_t *>(pack + (size_t)nb * 36)[blk] = qs;
        }
    }
}

// One float4 chunk per thread where the workgroup allows (the exact sum's
// per-thread share of terms stays small).
inline int norm_threads(int dim)
{
    const int n4 = dim / 4;
    int t = n4 <= kNormMaxThreads ? n4 : (n4 + kMaxChunks - 1) / kMaxChunks;
    t = (t + 63) / 64 * 64;
    return t < 64 ? 64 : t;
}

// dims up to 4*kNormMaxThreads: one float4 chunk per thread, terms in registers
inline bool norm_one_chunk(int dim) { return dim / 4 <= kNormMaxThreads; }

inline size_t norm_lds(int dim)
{
    if (norm_one_chunk(dim)) return sizeof(mrml_xsum::Shared4);
    return (size_t)dim * sizeof(float) + (((size_t)dim + 15) & ~(size_t)15) + sizeof(mrml_xsum::Shared);
}

}  // namespace

bool norm_dim_ok(int dim) { return dim > 0 && dim % 32 == 0 && dim <= 4 * kMaxChunks * kNormMaxThreads; }

// rms_norm by a group of 4 waves with K values per lane (exact_sum.h's group
// form, the sum the fused residual + GeGLU runs beside its weight stream):
// the same bits as rms_norm_kernel, for dim <= 256*K.  The pack goes through
// LDS into the 8-lanes-per-block layout of emit_q8.
constexpr int kGroupNormK = 9;

__host__ __device__ constexpr size_t group_norm_head() { return (sizeof(mrml_xsum::GroupShared) + 16 + 15) / 16 * 16; }
inline size_t group_norm_lds(int dim)
{
    return group_norm_head() + ((size_t)dim + 3) / 4 * 16 + (size_t)mrml_xsum::group_events(dim) * sizeof(float);
}

__global__ __launch_bounds__(256) void rms_norm_group_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                             float eps, float *__restrict__ out,
                                                             uint8_t *__restrict__ pack, int dim)
{
    const int polls = mrml_xsum::wait_polls();  // before the operand loads
    constexpr int K = kGroupNormK;
    x += (size_t)blockIdx.y * dim;  // row blockIdx.y of a batch (no pack then)
    if (out) out += (size_t)blockIdx.y * dim;
    extern __shared__ __align__(16) uint8_t lds[];
    auto *gs = reinterpret_cast<mrml_xsum::GroupShared *>(lds);
    uint32_t *ctr = reinterpret_cast<uint32_t *>(lds + sizeof(mrml_xsum::GroupShared));
    float *xn = reinterpret_cast<float *>(lds + group_norm_head());
    float *evl = xn + (dim + 3) / 4 * 4;
    const int wave = threadIdx.x >> 6, k0 = K * threadIdx.x;
    const float *wp = w ? w : x;  // unconditional loads
    float v[K], wv[K], sq[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const int k = k0 + i < dim ? k0 + i : dim - 1;
        v[i] = x[k];
        wv[i] = wp[k];
    }
#pragma unroll
    for (int i = 0; i < K; ++i) sq[i] = v[i] * v[i];
    if (threadIdx.x == 0) *ctr = 0u;
    __syncthreads();
    mrml_xsum::GroupSync sync{ctr, 0u, 4u, polls};
    const float scale = rms_scale(mrml_xsum::group_seq_sum_nonneg<K>(sq, dim, wave, sync, *gs, evl), dim, eps);
#pragma unroll
    for (int i = 0; i < K; ++i) {
        float o = v[i] * scale;
        if (w) o = o * wv[i];
        if (k0 + i < dim) {
            if (out) out[k0 + i] = o;
            xn[k0 + i] = o;
        }
    }
    if (!pack) return;
    __syncthreads();
    const int n4 = dim >> 2;
    const float4 *x4 = reinterpret_cast<const float4 *>(xn);
    for (int c0 = 0; c0 < n4; c0 += 256) {  // uniform
        const int c = c0 + threadIdx.x;
        emit_q8(x4[c < n4 ? c : n4 - 1], c, n4, pack, n4 >> 3);
    }
}

int launch_rms_norm(mrml_hip_ctx *ctx, const float *x, const float *w, float eps, float *out, void *pack, int dim,
                    int rows)
{
    if (rows > 1 && pack)
        return fail(ctx, MRML_HIP_E_INVALID, "rms_norm: a batch of rows writes no Q8_0 pack");
    const dim3 grid(1, rows);
    if (dim <= 256 * kGroupNormK && dim % 4 == 0) {
        hipLaunchKernelGGL(rms_norm_group_kernel, grid, dim3(256), group_norm_lds(dim), ctx->stream, x, w, eps, out,
                           (uint8_t *)pack, dim);
        return check_launch(ctx, "rms_norm_group_kernel");
    }
    if (norm_one_chunk(dim))
        hipLaunchKernelGGL(rms_norm_kernel<1>, grid, dim3(norm_threads(dim)), norm_lds(dim), ctx->stream, x, w, eps,
                           out, (uint8_t *)pack, dim);
    else
        hipLaunchKernelGGL(rms_norm_kernel<kMaxChunks>, grid, dim3(norm_threads(dim)), norm_lds(dim), ctx->stream, x,
                           w, eps, out, (uint8_t *)pack, dim);
    return check_launch(ctx, "rms_norm_kernel");
}

int launch_residual_rms_norm(mrml_hip_ctx *ctx, const float *t, const float *w_post, const float *h_in, float *h_out,
                             const float *w_next, float eps, float *xn, void *pack, int dim, int rows, bool fast,
                             void *gpack)
{
    if (gpack && !(xn && norm_one_chunk(dim) && dim % 32 == 0)) {  // the pack from xn, a launch of its own
        if (!xn) return fail(ctx, MRML_HIP_E_INVALID, "residual_rms_norm: a GEMM pack needs xn");
        if (int rc = launch_residual_rms_norm(ctx, t, w_post, h_in, h_out, w_next, eps, xn, pack, dim, rows, fast))
            return rc;
        return launch_gemm_pack_quantize(ctx, xn, gpack, dim, rows);
    }
    const dim3 grid(1, gpack ? gemm_groups(rows) * 32 : rows);
    uint8_t *gp = (uint8_t *)gpack;
    if (norm_one_chunk(dim) && fast)
        hipLaunchKernelGGL((residual_rms_norm_kernel<1, true>), grid, dim3(norm_threads(dim)), norm_lds(dim),
                           ctx->stream, t, w_post, h_in, h_out, w_next, eps, xn, (uint8_t *)pack, dim, gp, rows);
    else if (norm_one_chunk(dim))
        hipLaunchKernelGGL(residual_rms_norm_kernel<1>, grid, dim3(norm_threads(dim)), norm_lds(dim), ctx->stream, t,
                           w_post, h_in, h_out, w_next, eps, xn, (uint8_t *)pack, dim, gp, rows);
    else
        hipLaunchKernelGGL(residual_rms_norm_kernel<kMaxChunks>, grid, dim3(norm_threads(dim)), norm_lds(dim),
                           ctx->stream, t, w_post, h_in, h_out, w_next, eps, xn, (uint8_t *)pack, dim, gp, rows);
    return check_launch(ctx, "residual_rms_norm_kernel");
}

int launch_embedding(mrml_hip_ctx *ctx, const void *table, int type, const int32_t *d_token, int token, float scale,
                     float *h, const float *w_norm, float eps, float *xn, void *pack, int dim, int vocab, int rows)
{
    if (norm_one_chunk(dim))
        hipLaunchKernelGGL(embedding_kernel<1>, dim3(1, rows), dim3(norm_threads(dim)), norm_lds(dim), ctx->stream,
                           (const uint8_t *)table, type, d_token, token, scale, h, w_norm, eps, xn, (uint8_t *)pack, dim,
                           vocab);
    else
        hipLaunchKernelGGL(embedding_kernel<kMaxChunks>, dim3(1, rows), dim3(norm_threads(dim)), norm_lds(dim), ctx->stream,
                           (const uint8_t *)table, type, d_token, token, scale, h, w_norm, eps, xn, (uint8_t *)pack, dim,
                           vocab);
    return check_launch(ctx, "embedding_kernel");
}

int launch_rope_kv_f16(mrml_hip_ctx *ctx, float *qkv, uint16_t *k_cache, uint16_t *v_cache, const int32_t *d_pos,
                       int pos, int n_heads, int n_kv_heads, int head_dim, float base, float freq_scale, int capacity,
                       const float *table, int n_table, int rows, int cache_shift, const float *freqs)
{
    hipLaunchKernelGGL(rope_kv_f16_kernel, dim3(n_heads + 2 * n_kv_heads, rows), dim3(head_dim / 2), 0, ctx->stream, qkv,
                       k_cache, v_cache, d_pos, pos, n_heads, n_kv_heads, head_dim,
                       rope_args(table, n_table, base, freq_scale, freqs), capacity, cache_shift);
    return check_launch(ctx, "rope_kv_f16_kernel");
}

int launch_rope(mrml_hip_ctx *ctx, float *vec, int pos, int n_heads, int head_dim, float base, float freq_scale,
                const float *table, int n_table, const float *freqs)
{
    hipLaunchKernelGGL(rope_heads_kernel, dim3(n_heads), dim3(head_dim / 2), 0, ctx->stream, vec, pos, head_dim,
                       rope_args(table, n_table, base, freq_scale, freqs));
    return check_launch(ctx, "rope_heads_kernel");
}

int launch_add_rows(mrml_hip_ctx *ctx, const float *a, const float *b, float *out, int n)
{
    hipLaunchKernelGGL(add_rows_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, a, b, out, n);
    return check_launch(ctx, "add_rows_kernel");
}

int launch_swiglu_rows(mrml_hip_ctx *ctx, const float *g, const float *u, float *act, int n)
{
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, g, u, act, n,
                       (int)host_expf_fused());
    return check_launch(ctx, "swiglu_rows_kernel");
}

int attn_head_dim() { return kAttnHD; }
int attn_window_limit(int capacity, int sliding_window)
{
    return sliding_window > 0 && sliding_window < capacity ? sliding_window : capacity;
}
// 2^20 positions: past the reference's default max_context of 256000
// (model.rs:64-73); the scores take n_heads * capacity floats.
int attn_max_capacity() { return 1 << 20; }

size_t attn_scratch_bytes(int n_heads, int capacity) { return (size_t)n_heads * capacity * sizeof(float); }

// Softmax and weighted values of `rows` query rows (grid z), the LDS or the
// LONG form by capacity, V rows in format v_fmt.
static int launch_softmax_v(mrml_hip_ctx *ctx, const float *scores, const void *v_cache, float *out, void *pack,
                            const int32_t *d_pos, int n_past, int n_heads, int n_kv_heads, int capacity, int wlimit,
                            int rows = 1, int head_dim = kAttnHD, int v_fmt = 0)
{
    const dim3 grid(n_heads, head_dim / kSVD, rows), block(64 * kSVW);
    const uint8_t *v = reinterpret_cast<const uint8_t *>(v_cache);
    const int fe = (int)host_expf_fused();
#define SV_LAUNCH(LONG, VF)                                                                                          \
    hipLaunchKernelGGL((attn_softmax_v_kernel<LONG, VF>), grid, block, sv_lds(capacity), ctx->stream, scores, v,   \
                       d_pos, n_past, n_heads, n_kv_heads, head_dim, capacity, wlimit, fe, out, (uint8_t *)pack)
    const bool lg = sv_long(capacity);
    if (v_fmt == 1) {
        if (lg) SV_LAUNCH(true, 1); else SV_LAUNCH(false, 1);
    } else if (v_fmt == 2) {
        if (lg) SV_LAUNCH(true, 2); else SV_LAUNCH(false, 2);
    } else {
        if (lg) SV_LAUNCH(true, 0); else SV_LAUNCH(false, 0);
    }
#undef SV_LAUNCH
    return check_launch(ctx, "attn_softmax_v_kernel");
}

int launch_attn_decode_f16(mrml_hip_ctx *ctx, const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                           float *out, void *pack, const int32_t *d_pos, int n_past, int n_heads, int n_kv_heads,
                           float scale, int capacity, void *scratch, int sliding_window)
{
    float *scores = reinterpret_cast<float *>(scratch);
    const dim3 sgrid((capacity + kScoreP - 1) / kScoreP, n_kv_heads);
    const int wlimit = attn_window_limit(capacity, sliding_window);
    if (n_heads / n_kv_heads <= 4) {
        hipLaunchKernelGGL(attn_scores2_kernel<false>, sgrid, dim3(kScoreT), 0, ctx->stream, q,
                           const_cast<uint16_t *>(k_cache), (uint16_t *)nullptr, d_pos, n_past, n_heads, n_kv_heads,
                           scale, capacity, wlimit, RopeArgs{}, scores, 0);
        if (int rc = check_launch(ctx, "attn_scores2_kernel")) return rc;
    } else {
        hipLaunchKernelGGL(attn_scores_kernel, sgrid, dim3(64 * (n_heads / n_kv_heads)), 0, ctx->stream, q, k_cache,
                           d_pos, n_past, n_heads, n_kv_heads, scale, capacity, wlimit, scores, 0);
        if (int rc = check_launch(ctx, "attn_scores_kernel")) return rc;
    }
    return launch_softmax_v(ctx, scores, v_cache, out, pack, d_pos, n_past, n_heads, n_kv_heads, capacity, wlimit);
}

// Attention of `rows` queries at consecutive positions n_past0, n_past0+1, ...
// (the prefill of a chunk whose K/V rows are already in the cache): query row
// r starts r * q_stride floats into q (q_stride = the stacked q|k|v width
// when q is the projection itself); output row r (n_heads*head_dim f32) goes
// to out.  Each row's arithmetic is that of launch_attn_decode_f16 at its
// position with the same sliding window.  scratch holds rows * n_heads *
// capacity floats.  Groups of up to 8 query heads per kv head.
int launch_attn_rows_f16(mrml_hip_ctx *ctx, const float *q, int q_stride, const uint16_t *k_cache,
                         const uint16_t *v_cache, float *out, int n_past0, int rows, int n_heads, int n_kv_heads,
                         float scale, int capacity, void *scratch, int sliding_window)
{
    float *scores = reinterpret_cast<float *>(scratch);
    const int wlimit = attn_window_limit(capacity, sliding_window);
    // score tiles up to the widest row window (the host knows every row's position)
    const int span = std::min(wlimit, n_past0 + rows);
    const dim3 sgrid((span + kScoreP - 1) / kScoreP, n_kv_heads, rows);
    if (attn_rope_ok(n_heads, n_kv_heads) && (q_stride % 4 != 0 || ((uintptr_t)q & 15) != 0)) {
        // q rows that float4 reads cannot reach: one workgroup per row and tile
        hipLaunchKernelGGL(attn_scores2_kernel<false>, sgrid, dim3(kScoreT), 0, ctx->stream, q,
                           const_cast<uint16_t *>(k_cache), (uint16_t *)nullptr, (const int32_t *)nullptr, n_past0,
                           n_heads, n_kv_heads, scale, capacity, wlimit, RopeArgs{}, scores, q_stride);
        if (int rc = check_launch(ctx, "attn_scores2_kernel")) return rc;
    } else if (attn_rope_ok(n_heads, n_kv_heads)) {
        // positions tiled absolutely from row 0's window start to the last
        // row's position, 8 / G rows a workgroup
        const int g = n_heads / n_kv_heads, rb = kSRowsW / g;
        const int count0 = n_past0 + 1, t_lo = count0 > wlimit ? count0 - wlimit : 0, t_hi = n_past0 + rows - 1;
        const dim3 rgrid((unsigned)((t_hi - t_lo + kScoreP) / kScoreP), (unsigned)n_kv_heads,
                         (unsigned)((rows + rb - 1) / rb));
#define SCORES_ROWS(G)                                                                                          \
    hipLaunchKernelGGL(attn_scores_rows_kernel<G>, rgrid, dim3(64 * kSRowsW), 0, ctx->stream, q, q_stride,       \
                       k_cache, n_past0, rows, n_heads, n_kv_heads, scale, capacity, wlimit, t_lo, scores)
        switch (g) {
        case 1: SCORES_ROWS(1); break;
        case 2: SCORES_ROWS(2); break;
        case 3: SCORES_ROWS(3); break;
        default: SCORES_ROWS(4); break;
        }
#undef SCORES_ROWS
        if (int rc = check_launch(ctx, "attn_scores_rows_kernel")) return rc;
    } else {
        hipLaunchKernelGGL(attn_scores_kernel, sgrid, dim3(64 * (n_heads / n_kv_heads)), 0, ctx->stream, q, k_cache,
                           (const int32_t *)nullptr, n_past0, n_heads, n_kv_heads, scale, capacity, wlimit, scores,
                           q_stride);
        if (int rc = check_launch(ctx, "attn_scores_kernel")) return rc;
    }
    // the rows form where its dynamic LDS stays within 60 KiB; with the
    // kernel's static LDS (mrml_xsum::Shared, red, exp_tab: about 8.6 KB)
    // a launch takes up to about 69 KB, within gfx950's 160 KiB a workgroup
    if (span <= kRowsSvMax && n_heads / n_kv_heads <= kRowsSvG &&
        rows_sv_lds(n_heads / n_kv_heads, span) <= (size_t)60 << 10) {
#define ROWS_SV(G, S)                                                                                           \
    hipLaunchKernelGGL((attn_softmax_v_rows_kernel<G, S>), dim3(n_kv_heads, rows), dim3(kAttnHD),                \
                       rows_sv_lds(n_heads / n_kv_heads, span), ctx->stream, scores, v_cache, n_past0, n_heads,   \
                       n_kv_heads, capacity, wlimit, (int)host_expf_fused(), out, span)
        const bool sh = span <= 4 * kAttnHD;
        switch (n_heads / n_kv_heads) {
        case 1: if (sh) ROWS_SV(1, true); else ROWS_SV(1, false); break;
        case 2: if (sh) ROWS_SV(2, true); else ROWS_SV(2, false); break;
        case 3: if (sh) ROWS_SV(3, true); else ROWS_SV(3, false); break;
        default: if (sh) ROWS_SV(4, true); else ROWS_SV(4, false); break;
        }
#undef ROWS_SV
        return check_launch(ctx, "attn_softmax_v_rows_kernel");
    }
    return launch_softmax_v(ctx, scores, v_cache, out, nullptr, nullptr, n_past0, n_heads, n_kv_heads, capacity, wlimit,
                            rows);
}

// The decode step's attention with RoPE and the K/V append in the scores
// kernel: qkv is the raw stacked q|k|v vector.  Needs n_heads / n_kv_heads
// <= 4 (attn_rope_ok).
bool attn_rope_ok(int n_heads, int n_kv_heads) { return n_kv_heads > 0 && n_heads / n_kv_heads <= 4; }

int launch_attn_decode_rope_f16(mrml_hip_ctx *ctx, const float *qkv, uint16_t *k_cache, uint16_t *v_cache,
                                float *out, void *pack, const int32_t *d_pos, int n_past, int n_heads, int n_kv_heads,
                                float scale, int capacity, const float *table, int n_table, float base,
                                float freq_scale, void *scratch, const float *freqs, int sliding_window)
{
    float *scores = reinterpret_cast<float *>(scratch);
    const dim3 sgrid((capacity + kScoreP - 1) / kScoreP, n_kv_heads);
    const int wlimit = attn_window_limit(capacity, sliding_window);
    hipLaunchKernelGGL(attn_scores2_kernel<true>, sgrid, dim3(kScoreT), 0, ctx->stream, qkv, k_cache, v_cache, d_pos,
                       n_past, n_heads, n_kv_heads, scale, capacity, wlimit,
                       rope_args(table, n_table, base, freq_scale, freqs), scores, 0);
    if (int rc = check_launch(ctx, "attn_scores2_kernel")) return rc;
    return launch_softmax_v(ctx, scores, v_cache, out, pack, d_pos, n_past, n_heads, n_kv_heads, capacity, wlimit);
}

bool attn_any_ok(int n_heads, int n_kv_heads, int head_dim)
{
    return n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= kAnyMaxG && head_dim >= 32 &&
           head_dim <= kAnyMaxHD && head_dim % 32 == 0;
}

// The Gemma-2 shape the tuned kernels serve: head_dim 256, f16 rows, groups up to 8.
bool attn_tuned(int n_heads, int n_kv_heads, int head_dim, int k_fmt, int v_fmt)
{
    return head_dim == kAttnHD && k_fmt == 0 && v_fmt == 0 && n_kv_heads > 0 && n_heads / n_kv_heads <= 8;
}

int launch_attn_any(mrml_hip_ctx *ctx, const float *q, int q_stride, const void *k_cache, const void *v_cache,
                    float *out, void *pack, const int32_t *d_pos, int n_past0, int rows, int n_heads, int n_kv_heads,
                    int head_dim, int k_fmt, int v_fmt, float scale, int capacity, void *scratch, int sliding_window)
{
    float *scores = reinterpret_cast<float *>(scratch);
    const int wlimit = attn_window_limit(capacity, sliding_window);
    // score tiles up to the widest row window (every tile when the position is on the device)
    const int span = d_pos ? wlimit : std::min(wlimit, n_past0 + rows);
    const dim3 sgrid((span + kAnyP - 1) / kAnyP, n_kv_heads, rows);
    const size_t lds = attn_any_scores_lds(k_fmt, n_heads / n_kv_heads, head_dim);
    const uint8_t *kc = reinterpret_cast<const uint8_t *>(k_cache);
#define SC_LAUNCH(KF)                                                                                             \
    hipLaunchKernelGGL(attn_scores_any_kernel<KF>, sgrid, dim3(kAnyT), lds, ctx->stream, q, kc, d_pos, n_past0,  \
                       n_heads, n_kv_heads, head_dim, scale, capacity, wlimit, scores, q_stride)
    if (k_fmt == 1)
        SC_LAUNCH(1);
    else if (k_fmt == 2)
        SC_LAUNCH(2);
    else
        SC_LAUNCH(0);
#undef SC_LAUNCH
    if (int rc = check_launch(ctx, "attn_scores_any_kernel")) return rc;
    return launch_softmax_v(ctx, scores, v_cache, out, pack, d_pos, n_past0, n_heads, n_kv_heads, capacity, wlimit,
                            rows, head_dim, v_fmt);
}

int launch_rope_kv_any(mrml_hip_ctx *ctx, float *qkv, void *k_cache, void *v_cache, int pos, int n_heads,
                       int n_kv_heads, int head_dim, float base, float freq_scale, int capacity, const float *table,
                       int n_table, int rows, int cache_shift, int k_fmt, int v_fmt, const float *freqs)
{
    if (k_fmt == 0 && v_fmt == 0)
        return launch_rope_kv_f16(ctx, qkv, (uint16_t *)k_cache, (uint16_t *)v_cache, nullptr, pos, n_heads,
                                  n_kv_heads, head_dim, base, freq_scale, capacity, table, n_table, rows, cache_shift,
                                  freqs);
    // rotation only, then every K/V head stored in its cache's format
    if (int rc = launch_rope_kv_f16(ctx, qkv, nullptr, nullptr, nullptr, pos, n_heads, n_kv_heads, head_dim, base,
                                    freq_scale, capacity, table, n_table, rows, cache_shift, freqs))
        return rc;
    const dim3 grid(2 * n_kv_heads, rows);
    uint8_t *kc = reinterpret_cast<uint8_t *>(k_cache), *vc = reinterpret_cast<uint8_t *>(v_cache);
#define KV_LAUNCH(KF, VF)                                                                                    \
    hipLaunchKernelGGL((kv_append_any_kernel<KF, VF>), grid, dim3(64), 0, ctx->stream, qkv, kc, vc, pos,    \
                       n_heads, n_kv_heads, head_dim, capacity, cache_shift)
    switch (k_fmt * 3 + v_fmt) {
    case 1: KV_LAUNCH(0, 1); break;
    case 2: KV_LAUNCH(0, 2); break;
    case 3: KV_LAUNCH(1, 0); break;
    case 4: KV_LAUNCH(1, 1); break;
    case 5: KV_LAUNCH(1, 2); break;
    case 6: KV_LAUNCH(2, 0); break;
    case 7: KV_LAUNCH(2, 1); break;
    default: KV_LAUNCH(2, 2); break;
    }
#undef KV_LAUNCH
    return check_launch(ctx, "kv_append_any_kernel");
}

int attn_split_tiles(int capacity) { return (capacity + kSplitP - 1) / kSplitP; }

size_t attn_split_scratch_bytes(int n_heads, int capacity)
{
    return (size_t)n_heads * attn_split_tiles(capacity) * kSplitPart * sizeof(float);
}

int launch_attn_split_f16(mrml_hip_ctx *ctx, const float *qkv, uint16_t *k_cache, uint16_t *v_cache, float *out,
                          void *pack, const int32_t *d_pos, int n_past, int n_heads, int n_kv_heads, float scale,
                          int capacity, bool rope, const float *table, int n_table, float base, float freq_scale,
                          void *scratch, int sliding_window, const float *freqs)
{
    float *part = reinterpret_cast<float *>(scratch);
    const int tiles = attn_split_tiles(capacity), wlimit = attn_window_limit(capacity, sliding_window);
    const dim3 grid(tiles, n_kv_heads);
    const RopeArgs ra = rope_args(table, n_table, base, freq_scale, freqs);
    if (rope)
        hipLaunchKernelGGL(attn_split_kernel<true>, grid, dim3(kSplitT), 0, ctx->stream, qkv, k_cache, v_cache, d_pos,
                           n_past, n_heads, n_kv_heads, scale, capacity, wlimit, ra, part, tiles);
    else
        hipLaunchKernelGGL(attn_split_kernel<false>, grid, dim3(kSplitT), 0, ctx->stream, qkv, k_cache, v_cache,
                           d_pos, n_past, n_heads, n_kv_heads, scale, capacity, wlimit, ra, part, tiles);
    if (int rc = check_launch(ctx, "attn_split_kernel")) return rc;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads), dim3(kAttnHD), 0, ctx->stream, part, d_pos, n_past,
                       capacity, wlimit, tiles, n_heads, out, (uint8_t *)pack);
    return check_launch(ctx, "attn_combine_kernel");
}

hipError_t wait_guard_decode(int polls, uint32_t *timeouts) { return mrml_xsum::wait_guard_io(polls, timeouts); }

}  // namespace mrml
