// gemv_q8_q4k.hip -- batch-1 Q8_0 and Q4_K matrix-vector products and the
// greedy argmax, gfx950.  Same wave mapping and ordered DPP fold as the Q4_0
// kernels (one 16-lane DPP row per matrix row, 4 rows per wave); this file
// is compiled with -ffp-contract=off.

#include "device.h"
#include "internal.h"

namespace mrml {

namespace {


// Wave 0 of each workgroup copies the activation pack into LDS; the compute
// waves issue only their weight loads (see gemv_q4_0.hip).
__device__ __forceinline__ void stage_pack_wave(const uint8_t *src, uint8_t *lds, int nb)
{
    const int n16 = (nb * 40 + 15) >> 4;
    const uint4 *s = reinterpret_cast<const uint4 *>(src);
    uint4 *d = reinterpret_cast<uint4 *>(lds);
    for (int i = threadIdx.x; i < n16; i += 64) d[i] = s[i];
}

// ---- Q8_0 (quant.rs:563-577 semantics; model.rs:2842-2853 softcap) ---------
// Backend layout: quant plane [rows*nb][32 B], scale plane [rows*nb] f16.

// ODD: the matrix has an odd number of blocks, so the 4-byte word of the last
// scale would reach past the scale plane; scales are then read with 2-byte
// loads.
template <int ITERS, int WAVES, bool ODD>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q8_0_kernel(const uint8_t *__restrict__ w,
                                                                     const uint8_t *xpack,
                                                                     float *__restrict__ y, int rows, int nb,
                                                                     int softcap)
{
    extern __shared__ uint8_t lds[];
    if (threadIdx.x < 64) {
        stage_pack_wave(xpack, lds, nb);
        __syncthreads();
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int quad = blockIdx.x * WAVES + (threadIdx.x >> 6) - 1;
    const int row_raw = quad * 4 + (lane >> 4);
    const int row = row_raw < rows ? row_raw : rows - 1;
    const size_t nblk = (size_t)rows * nb;
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint16_t *dp = reinterpret_cast<const uint16_t *>(w + nblk * 32);
    const size_t base = (size_t)row * nb;

    // Scales are read as the 4-byte word holding them (see gemv_q4_0.hip);
    // tail lanes load a clamped in-bounds block and are masked in the fold.
    const uint32_t *dw = reinterpret_cast<const uint32_t *>(dp);
    uint4 w0[ITERS], w1[ITERS];
    uint32_t d[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        int b = it * 16 + j;
        b = b < nb ? b : nb - 1;
        w0[it] = qs[2 * (base + b)];
        w1[it] = qs[2 * (base + b) + 1];
        d[it] = ODD ? (uint32_t)dp[base + b] : dw[(base + b) >> 1];
    }
    __syncthreads();
    const int4 *aq = reinterpret_cast<const int4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + nb * 32);
    float s = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int bt = it * 16 + j;
        const int b = bt < nb ? bt : nb - 1;
        {
            const int4 a0 = aq[2 * b], a1 = aq[2 * b + 1];
            int32_t isum = sdot4(w0[it].x, (uint32_t)a0.x, 0);
            isum = sdot4(w0[it].y, (uint32_t)a0.y, isum);
            isum = sdot4(w0[it].z, (uint32_t)a0.z, isum);
            isum = sdot4(w0[it].w, (uint32_t)a0.w, isum);
            isum = sdot4(w1[it].x, (uint32_t)a1.x, isum);
            isum = sdot4(w1[it].y, (uint32_t)a1.y, isum);
            isum = sdot4(w1[it].z, (uint32_t)a1.z, isum);
            isum = sdot4(w1[it].w, (uint32_t)a1.w, isum);
            const size_t blk = base + b;
            const float tv = (float)isum * (f16_bits_to_f32((!ODD && (blk & 1)) ? d[it] >> 16 : d[it] & 0xffffu) * ad[b]);
            const float t = bt < nb ? tv : 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) s = fold16(s, t);
        }
    }
    if (j == 15 && row_raw < rows) y[row_raw] = softcap ? 30.0f * mrml_libm::tanhf(s / 30.0f) : s;
}

// ---- Q4_K (build-defined semantics over the GGUF super-block) ---------------
// Backend layout (repack_q4_k_kernel): quant plane [rows*nsb*8][16 B], one
// 16-byte run per 32-weight sub-block in Q4_0 nibble order, then the header
// plane [rows*nsb][16 B] = {f16 d, f16 dmin, 96-bit field of the 6-bit
// scales (bits 6j..) and mins (bits 48+6j..)}.  The rows then stream like
// Q4_0 rows of 8*nsb blocks: lane j of a 16-lane row owns sub-blocks
// 16*it + j (sub-block j & 7 of its super-block in every iteration), and the
// ordered DPP fold adds their terms in sub-block order (super-blocks, then
// sub-blocks, the oracle's order).  Term of a sub-block:
//   t = (float)isum * ((d * sc) * da) - (float)bsum * ((dmin * m) * da),
//   isum = sum q*a (q = 0..15), bsum = sum a (the activation block's sum),
// the integer dot on the split-nibble pack (stage_split_pack's KQ form: 8
// dot8 and 4 xor per sub-block).  The 8 lanes of a super-block share its
// header: each lane loads one 4-byte word of it (lane j: word j & 3, so
// every quad of lanes holds the whole header) and gets the other three by
// DPP quad broadcasts, which keeps the header in one register per iteration
// instead of four (occupancy).

template <int K>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, K | (K << 2) | (K << 4) | (K << 6), 0xf, 0xf, false);
}

template <int ITERS, int WAVES>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q4_k_kernel(const uint8_t *__restrict__ w,
                                                                     const uint8_t *xpack,
                                                                     float *__restrict__ y, int rows, int nsb)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int nb = nsb * 8;  // sub-blocks per row = activation blocks
    if (threadIdx.x < 64) {
        stage_split_pack<true, true>(xpack, lds, nb);
        __syncthreads();
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int quad = blockIdx.x * WAVES + (threadIdx.x >> 6) - 1;
    const int row_raw = quad * 4 + (lane >> 4);
    const int row = row_raw < rows ? row_raw : rows - 1;  // tail rows recompute the last row
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint32_t *hp = reinterpret_cast<const uint32_t *>(w + (size_t)rows * nb * 16);
    const size_t base = (size_t)row * nb, hbase = (size_t)row * nsb;
    const int sh_sc = 6 * (j & 7), sh_m = 16 + 6 * (j & 7);

    // every load of the row first; past the row end a clamped in-bounds
    // sub-block, masked out of the fold
    uint4 q[ITERS];
    uint32_t hw[ITERS];
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        int b = it * 16 + j;
        b = b < nb ? b : nb - 1;
        q[it] = qs[base + b];
        hw[it] = hp[(hbase + (b >> 3)) * 4 + (j & 3)];
    }
    __syncthreads();
    const uint4 *aq = reinterpret_cast<const uint4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + nb * 32);
    const int32_t *ac = reinterpret_cast<const int32_t *>(lds + nb * 36);
    const int32_t *as = reinterpret_cast<const int32_t *>(lds + nb * 40);
    float s = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int bt = it * 16 + j;
        const int b = bt < nb ? bt : nb - 1;
        const uint4 wq = q[it], lo = aq[2 * b], hi = aq[2 * b + 1];
        const int32_t isum = q4_0_isum_split(wq.x, wq.y, wq.z, wq.w, lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w,
                                             ac[b]);
        const uint32_t h0 = quad_bcast<0>(hw[it]), h1 = quad_bcast<1>(hw[it]), h2 = quad_bcast<2>(hw[it]),
                       h3 = quad_bcast<3>(hw[it]);
        const uint64_t f_sc = (uint64_t)h1 | ((uint64_t)h2 << 32), f_m = (uint64_t)h2 | ((uint64_t)h3 << 32);
        const uint32_t sc = (uint32_t)(f_sc >> sh_sc) & 63u, m = (uint32_t)(f_m >> sh_m) & 63u;
        const float d = f16_bits_to_f32(h0 & 0xffffu);
        const float dmin = f16_bits_to_f32(h0 >> 16);
        const float da = ad[b];
        const float ds = (d * (float)sc) * da;
        const float dm = (dmin * (float)m) * da;
        const float tv = (float)isum * ds - (float)as[b] * dm;
        const float t = bt < nb ? tv : 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) s = fold16(s, t);
    }
    if (j == 15 && row_raw < rows) y[row_raw] = s;
}

// ---- argmax (lowest index on ties, NaN never wins) ---------------------------

__device__ __forceinline__ bool better(float av, int ai, float bv, int bi)
{
    const bool an = av != av, bn = bv != bv;
    if (an || bn) return (an && bn) ? ai < bi : bn;
    return av > bv || (av == bv && ai < bi);
}

__device__ __forceinline__ void block_best(float &v, int &i)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(i, off, 64);
        if (better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    __shared__ float sv[16];
    __shared__ int si[16];
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wave] = v; si[wave] = i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < nw; ++k)
            if (better(sv[k], si[k], v, i)) { v = sv[k]; i = si[k]; }
    }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *__restrict__ x, int n,
                                                             float *__restrict__ pv, int *__restrict__ pi)
{
    float v = __builtin_nanf("");
    int i = 0x7fffffff;
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < n; k += gridDim.x * blockDim.x) {
        const float xv = x[k];
        if (better(xv, k, v, i)) { v = xv; i = k; }
    }
    block_best(v, i);
    if (threadIdx.x == 0) { pv[blockIdx.x] = v; pi[blockIdx.x] = i; }
}

// With `state` = {token, pos} (device), also advances a decode loop kept on
// the device: hist[pos] = the argmax (when pos < hist_cap); pos += 1; token =
// prompt[pos] while pos < prompt_len (prefill), else the argmax.
__global__ __launch_bounds__(256) void argmax_final_kernel(const float *__restrict__ pv, const int *__restrict__ pi,
                                                           int parts, int32_t *__restrict__ out,
                                                           int32_t *__restrict__ state, int32_t *__restrict__ hist,
                                                           int hist_cap, const int32_t *__restrict__ prompt,
                                                           int prompt_len)
{
    float v = __builtin_nanf("");
    int i = 0x7fffffff;
    for (int k = threadIdx.x; k < parts; k += blockDim.x)
        if (better(pv[k], pi[k], v, i)) { v = pv[k]; i = pi[k]; }
    block_best(v, i);
    if (threadIdx.x == 0) {
        if (out) *out = i;
        if (state) {
            const int cur = state[1];
            if (hist && cur >= 0 && cur < hist_cap) hist[cur] = i;
            const int pos = cur + 1;
            state[0] = (prompt && pos < prompt_len) ? prompt[pos] : i;
            state[1] = pos;
        }
    }
}

inline int waves_for(int rows) { return rows >= 8192 ? 4 : (rows >= 2048 ? 2 : 1); }

// The smallest compiled iteration count >= iters (iterations past a row's
// last block are masked, so a larger instance gives the same result), or 0.
inline int iters_instance(int iters)
{
    static const int kInst[] = {1, 2, 3, 4, 5, 6, 8, 9, 12, 16, 18, 20};
    for (int v : kInst)
        if (v >= iters) return v;
    return 0;
}

#define MRML_DISPATCH_WAVES(WAVES_VAL, BODY)                 \
    switch (WAVES_VAL) {                                     \
    case 1: { constexpr int WV = 1; BODY; } break;           \
    case 2: { constexpr int WV = 2; BODY; } break;           \
    default: { constexpr int WV = 4; BODY; } break;          \
    }

}  // namespace

int launch_gemv_q8_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols,
                     int32_t softcap)
{
    const int nb = cols / 32;
    const bool odd = (((int64_t)rows * nb) & 1) != 0;
    const int iters = (nb + 15) / 16;
    const int waves = waves_for(rows);
    const dim3 grid(((rows + 3) / 4 + waves - 1) / waves);
    const size_t lds = act_pack_bytes(nb);
#define Q8_CASE(N)                                                                                           \
    case N:                                                                                                  \
        MRML_DISPATCH_WAVES(waves, {                                                                         \
            if (odd)                                                                                         \
                hipLaunchKernelGGL((gemv_q8_0_kernel<N, WV, true>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,   \
                                   (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb, softcap);       \
            else                                                                                             \
                hipLaunchKernelGGL((gemv_q8_0_kernel<N, WV, false>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,  \
                                   (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb, softcap);       \
        });                                                                                                  \
        break;
    switch (iters_instance(iters)) {
        Q8_CASE(1) Q8_CASE(2) Q8_CASE(3) Q8_CASE(4) Q8_CASE(5) Q8_CASE(6) Q8_CASE(8) Q8_CASE(9)
        Q8_CASE(12) Q8_CASE(16) Q8_CASE(18) Q8_CASE(20)
    default:
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "q8_0 matvec: cols=%d has no kernel instance", cols);
    }
#undef Q8_CASE
    return check_launch(ctx, "gemv_q8_0_kernel");
}

int launch_gemv_q4_k(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols)
{
    const int nsb = cols / 256, nb = nsb * 8;
    const int iters = (nb + 15) / 16;
    if (nb > kStageMax)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "q4_k matvec: cols=%d above %d", cols, kStageMax * 32);
    const int waves = waves_for(rows);
    const dim3 grid(((rows + 3) / 4 + waves - 1) / waves);
    const size_t lds = (size_t)nb * 44;  // split-nibble pack with block sums (stage_split_pack, KQ)
#define QK_CASE(N)                                                                                           \
    case N:                                                                                                  \
        MRML_DISPATCH_WAVES(waves, {                                                                         \
            hipLaunchKernelGGL((gemv_q4_k_kernel<N, WV>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,             \
                               (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nsb);                   \
        });                                                                                                  \
        break;
    switch (iters_instance(iters)) {
        QK_CASE(1) QK_CASE(2) QK_CASE(3) QK_CASE(4) QK_CASE(5) QK_CASE(6) QK_CASE(8) QK_CASE(9) QK_CASE(12)
        QK_CASE(16) QK_CASE(18) QK_CASE(20)
    default:
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "q4_k matvec: cols=%d has no kernel instance", cols);
    }
#undef QK_CASE
    return check_launch(ctx, "gemv_q4_k_kernel");
}

int argmax_parts(int32_t n)
{
    const int parts = (n + 2047) / 2048;
    return parts > 1024 ? 1024 : parts;
}

int launch_argmax_step(mrml_hip_ctx *ctx, const float *x, int32_t n, int32_t *out, void *scratch, int32_t *state,
                       int32_t *hist, int hist_cap, const int32_t *prompt, int prompt_len)
{
    const int parts = argmax_parts(n);
    float *pv = reinterpret_cast<float *>(scratch);
    int *pi = reinterpret_cast<int *>(reinterpret_cast<uint8_t *>(scratch) + (size_t)parts * 4);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts), dim3(256), 0, ctx->stream, x, n, pv, pi);
    int rc = check_launch(ctx, "argmax_partial_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, ctx->stream, pv, pi, parts, out, state, hist,
                       hist_cap, prompt, prompt_len);
    return check_launch(ctx, "argmax_final_kernel");
}

int launch_argmax_f32(mrml_hip_ctx *ctx, const float *x, int32_t n, int32_t *out)
{
    void *ws = workspace(ctx, (size_t)argmax_parts(n) * 8);
    if (!ws) return MRML_HIP_E_ALLOC;
    return launch_argmax_step(ctx, x, n, out, ws, nullptr, nullptr, 0, nullptr, 0);
}

}  // namespace mrml
