// gemv_q8_q4k.hip -- batch-1 Q8_0 and Q4_K matrix-vector products and the
// greedy argmax, gfx950.  Same wave mapping and ordered DPP fold as the Q4_0
// kernels (one 16-lane DPP row per matrix row, 4 rows per wave); this file
// is compiled with -ffp-contract=off.

#include "device.h"
#include "internal.h"

namespace mrml {

namespace {

constexpr uint32_t kNib = 0x0F0F0F0Fu;

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

template <int ITERS, int WAVES>
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
        d[it] = dw[(base + b) >> 1];
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
            const float tv = (float)isum * (f16_bits_to_f32((blk & 1) ? d[it] >> 16 : d[it] & 0xffffu) * ad[b]);
            const float t = bt < nb ? tv : 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) s = fold16(s, t);
        }
    }
    if (j == 15 && row_raw < rows) y[row_raw] = softcap ? 30.0f * mrml_libm::tanhf(s / 30.0f) : s;
}

// ---- Q4_K (build-defined semantics over the GGUF super-block) ---------------
// Backend layout: quant plane [rows*nsb][128 B], header plane [rows*nsb][16 B]
// = {f16 d, f16 dmin, u8 scales[12]}.  A lane owns one 32-byte quarter c of a
// super-block: the low nibbles are sub-block 2c, the high nibbles 2c+1.
// Since 16 lanes cover 4 super-blocks, c = j & 3 is fixed per lane.

__device__ __forceinline__ uint32_t hdr_byte(const uint4 &h, int i)
{
    const uint32_t word = (i < 4) ? h.x : (i < 8) ? h.y : (i < 12) ? h.z : h.w;
    return (word >> ((i & 3) * 8)) & 0xffu;
}

// GGUF get_scale_min_k4 for sub-block jj (0..7); scales start at header byte 4.
__device__ __forceinline__ void q4k_scale_min(const uint4 &h, int jj, uint32_t &sc, uint32_t &m)
{
    if (jj < 4) {
        sc = hdr_byte(h, 4 + jj) & 63u;
        m = hdr_byte(h, 8 + jj) & 63u;
    } else {
        sc = (hdr_byte(h, 8 + jj) & 0x0fu) | ((hdr_byte(h, jj) >> 6) << 4);
        m = (hdr_byte(h, 8 + jj) >> 4) | ((hdr_byte(h, 4 + jj) >> 6) << 4);
    }
}

template <int ITERS, int WAVES>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q4_k_kernel(const uint8_t *__restrict__ w,
                                                                     const uint8_t *xpack,
                                                                     float *__restrict__ y, int rows, int nsb)
{
    extern __shared__ uint8_t lds[];
    if (threadIdx.x < 64) {
        stage_pack_wave(xpack, lds, nsb * 8);
        __syncthreads();
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15, c = j & 3;
    const int quad = blockIdx.x * WAVES + (threadIdx.x >> 6) - 1;
    const int row_raw = quad * 4 + (lane >> 4);
    const int row = row_raw < rows ? row_raw : rows - 1;
    const size_t nsbt = (size_t)rows * nsb;
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint4 *hp = reinterpret_cast<const uint4 *>(w + nsbt * 128);
    const size_t base = (size_t)row * nsb;
    const int nchunks = nsb * 4;
    const int nb = nsb * 8;

    uint4 w0[ITERS], w1[ITERS], h[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        int g = it * 16 + j;
        g = g < nchunks ? g : nchunks - 4 + c;  // tail lanes: an in-bounds chunk, masked below
        const size_t sbi = base + (size_t)(g >> 2);
        w0[it] = qs[sbi * 8 + 2 * c];
        w1[it] = qs[sbi * 8 + 2 * c + 1];
        h[it] = hp[sbi];
    }
    __syncthreads();
    const int4 *aq = reinterpret_cast<const int4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + nb * 32);
    const int32_t *as = reinterpret_cast<const int32_t *>(lds + nb * 36);
    float s = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int gt = it * 16 + j;
        const int g = gt < nchunks ? gt : nchunks - 4 + c;
        float te, to;
        {
            const int be = (g >> 2) * 8 + 2 * c;  // activation block of sub-block 2c
            const int4 e0 = aq[2 * be], e1 = aq[2 * be + 1];
            const int4 o0 = aq[2 * be + 2], o1 = aq[2 * be + 3];
            const uint4 q0 = w0[it], q1 = w1[it];
            int32_t ie = sdot4(q0.x & kNib, (uint32_t)e0.x, 0);
            ie = sdot4(q0.y & kNib, (uint32_t)e0.y, ie);
            ie = sdot4(q0.z & kNib, (uint32_t)e0.z, ie);
            ie = sdot4(q0.w & kNib, (uint32_t)e0.w, ie);
            ie = sdot4(q1.x & kNib, (uint32_t)e1.x, ie);
            ie = sdot4(q1.y & kNib, (uint32_t)e1.y, ie);
            ie = sdot4(q1.z & kNib, (uint32_t)e1.z, ie);
            ie = sdot4(q1.w & kNib, (uint32_t)e1.w, ie);
            int32_t io = sdot4((q0.x >> 4) & kNib, (uint32_t)o0.x, 0);
            io = sdot4((q0.y >> 4) & kNib, (uint32_t)o0.y, io);
            io = sdot4((q0.z >> 4) & kNib, (uint32_t)o0.z, io);
            io = sdot4((q0.w >> 4) & kNib, (uint32_t)o0.w, io);
            io = sdot4((q1.x >> 4) & kNib, (uint32_t)o1.x, io);
            io = sdot4((q1.y >> 4) & kNib, (uint32_t)o1.y, io);
            io = sdot4((q1.z >> 4) & kNib, (uint32_t)o1.z, io);
            io = sdot4((q1.w >> 4) & kNib, (uint32_t)o1.w, io);
            const float d = f16_bits_to_f32(h[it].x & 0xffffu);
            const float dmin = f16_bits_to_f32(h[it].x >> 16);
            uint32_t sc, m;
            q4k_scale_min(h[it], 2 * c, sc, m);
            {
                const float da = ad[be];
                const float ds = (d * (float)sc) * da;
                const float dm = (dmin * (float)m) * da;
                te = (float)ie * ds - (float)as[be] * dm;
            }
            q4k_scale_min(h[it], 2 * c + 1, sc, m);
            {
                const float da = ad[be + 1];
                const float ds = (d * (float)sc) * da;
                const float dm = (dmin * (float)m) * da;
                to = (float)io * ds - (float)as[be + 1] * dm;
            }
        }
        te = gt < nchunks ? te : 0.0f;
        to = gt < nchunks ? to : 0.0f;
        // Lane k's pair (t_{2c}, t_{2c+1}) joins the running sum at step k.
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            s = dpp_ror1(s) + te;
            s = s + to;
        }
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
    if (((int64_t)rows * nb) & 1)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED,
                    "q8_0 matvec: rows*cols/32 = %lld is odd (needs cols %% 64 == 0 or even rows)",
                    (long long)rows * nb);
    const int iters = (nb + 15) / 16;
    const int waves = waves_for(rows);
    const dim3 grid(((rows + 3) / 4 + waves - 1) / waves);
    const size_t lds = act_pack_bytes(nb);
#define Q8_CASE(N)                                                                                           \
    case N:                                                                                                  \
        MRML_DISPATCH_WAVES(waves, {                                                                         \
            hipLaunchKernelGGL((gemv_q8_0_kernel<N, WV>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,             \
                               (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb, softcap);           \
        });                                                                                                  \
        break;
    switch (iters) {
        Q8_CASE(1) Q8_CASE(2) Q8_CASE(3) Q8_CASE(4) Q8_CASE(5) Q8_CASE(6) Q8_CASE(8) Q8_CASE(9)
        Q8_CASE(12) Q8_CASE(16) Q8_CASE(18)
    default:
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "q8_0 matvec: cols=%d has no kernel instance", cols);
    }
#undef Q8_CASE
    return check_launch(ctx, "gemv_q8_0_kernel");
}

int launch_gemv_q4_k(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols)
{
    const int nsb = cols / 256;
    const int iters = (nsb * 4 + 15) / 16;
    const int waves = waves_for(rows);
    const dim3 grid(((rows + 3) / 4 + waves - 1) / waves);
    const size_t lds = act_pack_bytes(nsb * 8);
#define QK_CASE(N)                                                                                           \
    case N:                                                                                                  \
        MRML_DISPATCH_WAVES(waves, {                                                                         \
            hipLaunchKernelGGL((gemv_q4_k_kernel<N, WV>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,             \
                               (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nsb);                   \
        });                                                                                                  \
        break;
    switch (iters) {
        QK_CASE(1) QK_CASE(2) QK_CASE(3) QK_CASE(4) QK_CASE(5) QK_CASE(6) QK_CASE(8) QK_CASE(9)
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
