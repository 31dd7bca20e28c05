// norm_block.h -- RMSNorm pieces shared by the norm kernels and by the
// matvec kernels that run the Gemma-2 sandwich residual ahead of their rows.
// Values are held as float4 chunks c = threadIdx.x + k*blockDim; the sum of
// squares is the reference's sequential f32 loop, evaluated in parallel
// (exact_sum.h).
#pragma once

#include "device.h"
#include "exact_sum.h"

namespace mrml {

__device__ __forceinline__ float4 scale4(float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }
__device__ __forceinline__ float4 mul4(float4 a, float4 b)
{
    return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}
__device__ __forceinline__ float4 add4(float4 a, float4 b)
{
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 sq4(float4 a) { return make_float4(a.x * a.x, a.y * a.y, a.z * a.z, a.w * a.w); }


// Sum of squares of the values held in v (chunks c = tid + k*blockDim), in
// index order from +0 (ops.rs:24-79), bit for bit: the sequential f32 sum
// evaluated in parallel (exact_sum.h).  With one chunk per thread the terms
// stay in registers and `lds` holds an mrml_xsum::Shared4; otherwise they are
// staged in LDS: n4*4 floats, n4*4 flag bytes (16-byte aligned end), then an
// mrml_xsum::Shared.
//
// FAST (the decode step's tolerance path): a deterministic tree sum instead
// (exact_sum.h's block_tree_sum; needs CH == 1), the first floats of lds as
// its scratch.
template <int CH, bool FAST = false>
__device__ float block_seq_sum_sq(const float4 (&v)[CH], int n4, float *lds)
{
    if constexpr (FAST) {
        static_assert(CH == 1, "one chunk per thread");
        const int c = threadIdx.x;
        const float4 q = sq4(v[0]);
        return mrml_xsum::block_tree_sum(c < n4 ? (q.x + q.y) + (q.z + q.w) : 0.0f, lds);
    }
    if constexpr (CH == 1) {
        auto *x = reinterpret_cast<mrml_xsum::Shared4 *>(lds);
        return mrml_xsum::block_seq_sum_nonneg4(sq4(v[0]), n4 * 4, *x);
    }
    float4 *sq = reinterpret_cast<float4 *>(lds);
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        const int c = threadIdx.x + k * blockDim.x;
        if (c < n4) sq[c] = sq4(v[k]);
    }
    __syncthreads();
    uint8_t *flags = reinterpret_cast<uint8_t *>(lds + n4 * 4);
    auto *x = reinterpret_cast<mrml_xsum::Shared *>(flags + ((n4 * 4 + 15) & ~15));
    return mrml_xsum::block_seq_sum_nonneg(lds, n4 * 4, flags, *x);
}

// ops.rs:24-79: mean = sum/dim, scale = 1/sqrt(mean + eps) (IEEE sqrt and
// divide: hipcc's defaults are correctly rounded).
__device__ __forceinline__ float rms_scale(float sum_sq, int dim, float eps)
{
    const float mean = sum_sq / (float)dim;
    return 1.0f / sqrtf(mean + eps);
}

// Q8_0 pack of the value chunk c (values 4c..4c+3); 8 consecutive threads
// hold one block.  SPLIT writes the split-nibble form the Q4_0 kernels read
// from LDS (device.h; the sum plane then holds c).  Every lane of the wave
// must call this.
template <bool SPLIT = false>
__device__ __forceinline__ void emit_q8(float4 v, int c, int n4, uint8_t *pack, int nb)
{
    uint32_t dbits;
    int s;
    uint32_t q = q8_0_block8x4(v, dbits, s);
    if constexpr (SPLIT) q = q8_split8(q, c & 7, s);
    if (c < n4) {
        reinterpret_cast<uint32_t *>(pack)[c] = q;
        if ((c & 7) == 0) {
            reinterpret_cast<float *>(pack + (size_t)nb * 32)[c >> 3] = f16_bits_to_f32(dbits);
            reinterpret_cast<int32_t *>(pack + (size_t)nb * 36)[c >> 3] = s;
        }
    }
}

// Loads the weight chunks of this thread (w nullable: no load), issued
// with the kernel's other loads so none waits behind the norm's sums.
template <int CH>
__device__ __forceinline__ void load_w(const float *w, float4 (&wv)[CH], int n4)
{
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        const int c = threadIdx.x + k * blockDim.x;
        wv[k] = w ? w4[c < n4 ? c : 0] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    }
}

// out = (x * scale) * w per value (has_w false: no weight), stored to out
// (nullable) and as a Q8_0 pack (nullable; SPLIT: split-nibble form).
template <int CH, bool SPLIT = false>
__device__ __forceinline__ void norm_store(const float4 (&v)[CH], float scale, const float4 (&wv)[CH], bool has_w,
                                           float *out, uint8_t *pack, int n4)
{
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        if (k * (int)blockDim.x >= n4) break;  // uniform
        const int c = threadIdx.x + k * blockDim.x;
        float4 o = scale4(v[k], scale);
        if (has_w) o = mul4(o, wv[k]);
        if (out && c < n4) reinterpret_cast<float4 *>(out)[c] = o;
        if (pack) emit_q8<SPLIT>(o, c, n4, pack, n4 >> 3);
    }
}

// Operands of the Gemma-2 sandwich residual for this thread's float4 chunk
// (c = threadIdx.x, dim <= 4*blockDim).
struct ResidualOps {
    float4 t, h, wp, wn;
};

__device__ __forceinline__ ResidualOps residual_load(const float *__restrict__ t, const float *__restrict__ w_post,
                                                     const float *__restrict__ h_in, const float *__restrict__ w_next,
                                                     int n4)
{
    const float4 one4 = make_float4(1.0f, 1.0f, 1.0f, 1.0f), zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int c = threadIdx.x, cc = c < n4 ? c : 0;
    // four unconditional loads (a missing weight reads t and is replaced),
    // so no load sits in a branch of its own
    const float4 tv = reinterpret_cast<const float4 *>(t)[cc];
    const float4 hv = reinterpret_cast<const float4 *>(h_in)[cc];
    const float4 pv = reinterpret_cast<const float4 *>(w_post ? w_post : t)[cc];
    const float4 nv = reinterpret_cast<const float4 *>(w_next ? w_next : t)[cc];
    ResidualOps r;
    r.t = c < n4 ? tv : zero4;
    r.h = hv;
    r.wp = w_post ? pv : one4;
    r.wn = w_next ? nv : one4;
    return r;
}

// The sandwich-norm residual of a Gemma-2 block followed by the next block's
// pre-norm (the per-layer order of model.rs:1185-2260), one chunk per thread:
//   h_out = h_in + rms_norm(t, w_post)          (h_out nullable: not stored)
//   xn    = rms_norm(h_out, w_next)             -> xn (nullable) and its Q8_0 pack (nullable)
// Every thread of the workgroup calls it.  t is this thread's chunk of t;
// fetch(0), fetch(1), fetch(2) return its chunks of h_in, w_post and w_next
// when they are needed (registers, or LDS where a kernel parks them to keep
// registers free).  The pack may be in LDS; the caller synchronises before
// reading it.  h_out may equal h_in (each thread reads its chunk before
// writing it) only when no other workgroup reads h_in.  SPLIT: the pack is
// written in split-nibble form.
template <bool SPLIT = false, bool FAST = false, class Fetch>
__device__ __forceinline__ void residual_norm1(float4 t, Fetch fetch, bool has_wpost, bool has_wnext, float eps,
                                               float *h_out, float *xn, uint8_t *pack, int dim,
                                               mrml_xsum::Shared4 &x)
{
    const int n4 = dim >> 2, c = threadIdx.x;
    float4 v[1] = {t};
    const float s1 = rms_scale(block_seq_sum_sq<1, FAST>(v, n4, reinterpret_cast<float *>(&x)), dim, eps);
    float4 tn = scale4(t, s1);
    if (has_wpost) tn = mul4(tn, fetch(1));
    const float4 hn = add4(fetch(0), tn);
    if (h_out && c < n4) reinterpret_cast<float4 *>(h_out)[c] = hn;
    if (!xn && !pack) return;
    v[0] = c < n4 ? hn : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 wv[1] = {fetch(2)};
    norm_store<1, SPLIT>(v, rms_scale(block_seq_sum_sq<1, FAST>(v, n4, reinterpret_cast<float *>(&x)), dim, eps),
                         wv, has_wnext, xn, pack, n4);
}

template <bool SPLIT = false, bool FAST = false>
__device__ __forceinline__ void residual_norm1(const ResidualOps &r, bool has_wpost, bool has_wnext, float eps,
                                               float *h_out, float *xn, uint8_t *pack, int dim,
                                               mrml_xsum::Shared4 &x)
{
    residual_norm1<SPLIT, FAST>(r.t, [&](int k) { return k == 0 ? r.h : (k == 1 ? r.wp : r.wn); }, has_wpost,
                                has_wnext, eps, h_out, xn, pack, dim, x);
}

// Waits for this wave's outstanding global loads (s_waitcnt vmcnt(0), other
// counters untouched), through the builtin so the compiler's wait
// bookkeeping sees it.
__device__ __forceinline__ void wait_vm_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

}  // namespace mrml
