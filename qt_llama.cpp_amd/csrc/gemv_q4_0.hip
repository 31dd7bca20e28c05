// gemv_q4_0.hip -- batch-1 Q4_0 x Q8_0 matrix-vector products for gfx950.
//
// Semantics (crates/mrml-tensor/src/quant.rs:335-369, ops.rs:221-260):
//   isum_b = sum_i ((qs&15)-8)*a[i] + ((qs>>4)-8)*a[i+16]       exact int32
//   y[r]   = (...((0 + isum_0*(dw_0*da_0)) + isum_1*(dw_1*da_1)) ...)
// in block order, each product and each sum rounded separately (this file is
// compiled with -ffp-contract=off), so y is bit-identical to the CPU path.
//
// Mapping: one 64-lane wave owns 4 rows; the 16 lanes of a DPP row own one
// matrix row and take 16 consecutive blocks per iteration (lane j -> block
// 16*it + j).  In the backend layout a lane's block is one 16-byte load and
// the 16 lanes of a row read 256 contiguous bytes, so every load instruction
// is 4 fully used 256-byte segments.  All of a lane's weight loads are issued
// before any is consumed; they return in order, so the in-order fold starts
// on the first bytes to arrive.
//   isum: 8 v_dot4_i32_i8 on (nibbles, int8 activations) minus 8*sum(a).
//   fold: 16 row_ror:1 DPP adds per iteration; after step k lane k holds the
//         running sum through block 16*it+k, lane 15 ends with the row result.
// The activation pack (int8 quants, f32 scales, int32 sums) is staged once per
// workgroup in LDS.

#include "device.h"
#include "internal.h"

namespace mrml {

namespace {

constexpr uint32_t kNib = 0x0F0F0F0Fu;

// Activation pack staging.  Wave 0 of every workgroup only copies the pack
// (nb*40 bytes, 16-byte aligned) into LDS; the compute waves issue nothing
// but their own weight loads, so each of their in-order waits covers exactly
// the weight bytes it consumes and the fold starts on the first to arrive.
__device__ __forceinline__ void stage_pack_wave(const uint8_t *src, uint8_t *lds, int nb)
{
    const int n16 = (nb * 40 + 15) >> 4;
    const uint4 *s = reinterpret_cast<const uint4 *>(src);
    uint4 *d = reinterpret_cast<uint4 *>(lds);
    for (int i = threadIdx.x; i < n16; i += 64) d[i] = s[i];
}

// Exact integer block dot of one Q4_0 block (16 packed bytes) with the
// matching Q8_0 activation block (32 int8 in LDS) and its quant sum.
__device__ __forceinline__ int32_t q4_0_isum(uint4 w, const int4 *aq, int32_t asum)
{
    const int4 a0 = aq[0], a1 = aq[1];
    int32_t s = sdot4(w.x & kNib, (uint32_t)a0.x, 0);
    s = sdot4(w.y & kNib, (uint32_t)a0.y, s);
    s = sdot4(w.z & kNib, (uint32_t)a0.z, s);
    s = sdot4(w.w & kNib, (uint32_t)a0.w, s);
    s = sdot4((w.x >> 4) & kNib, (uint32_t)a1.x, s);
    s = sdot4((w.y >> 4) & kNib, (uint32_t)a1.y, s);
    s = sdot4((w.z >> 4) & kNib, (uint32_t)a1.z, s);
    s = sdot4((w.w >> 4) & kNib, (uint32_t)a1.w, s);
    return s - 8 * asum;  // nibble offset: sum (q-8)*a = sum q*a - 8*sum a
}

// Per-lane register block of one matrix row: ITERS blocks of 16-byte quants
// and, per block, the 32-bit word of the scale plane holding its f16 scale
// (two neighbouring blocks share a word; a 4-byte load keeps each scale in
// its own register so no load is consumed before the fold needs it).
// Blocks past the row end load a clamped in-bounds address and are masked
// out of the fold.
template <int ITERS>
struct RowRegs {
    uint4 w[ITERS];
    uint32_t d[ITERS];
};

template <int ITERS>
__device__ __forceinline__ void load_row(RowRegs<ITERS> &r, const uint4 *__restrict__ qs,
                                         const uint16_t *__restrict__ dp, size_t base, int nb, int j)
{
    const uint32_t *dw = reinterpret_cast<const uint32_t *>(dp);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        int b = it * 16 + j;
        b = b < nb ? b : nb - 1;
        r.w[it] = qs[base + b];
        r.d[it] = dw[(base + b) >> 1];
    }
}

__device__ __forceinline__ uint32_t scale_bits(uint32_t word, size_t blk) { return (blk & 1) ? word >> 16 : word & 0xffffu; }

// Ordered fold of one row held as RowRegs; result valid in lane 15 of the
// DPP row.  Masked tail blocks contribute +0, which leaves a running sum
// unchanged (the running sum is never -0: it starts at +0 and
// round-to-nearest never produces -0 from a sum with a +0 operand).
template <int ITERS>
__device__ __forceinline__ float fold_row(const RowRegs<ITERS> &r, const uint8_t *lds, size_t base, int nb, int j)
{
    const int4 *aq = reinterpret_cast<const int4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + nb * 32);
    const int32_t *as = reinterpret_cast<const int32_t *>(lds + nb * 36);
    float s = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        // Computed unconditionally (tail lanes hold a clamped, valid block) so
        // the compiler has no conditional block to sink the weight load into.
        const int b = it * 16 + j;
        const int bc = b < nb ? b : nb - 1;
        const int32_t isum = q4_0_isum(r.w[it], aq + 2 * bc, as[bc]);
        const float tv = (float)isum * (f16_bits_to_f32(scale_bits(r.d[it], base + bc)) * ad[bc]);
        const float t = b < nb ? tv : 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) s = fold16(s, t);
    }
    return s;
}

// ---- plain matvec ----------------------------------------------------------

template <int ITERS, int WAVES>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q4_0_kernel(const uint8_t *__restrict__ w,
                                                                     const uint8_t *xpack,
                                                                     float *__restrict__ y, int rows, int nb)
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
    const int row = row_raw < rows ? row_raw : rows - 1;  // tail rows recompute the last row
    const size_t nblk = (size_t)rows * nb;
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint16_t *dp = reinterpret_cast<const uint16_t *>(w + nblk * 16);

    RowRegs<ITERS> r;
    load_row<ITERS>(r, qs, dp, (size_t)row * nb, nb, j);
    __syncthreads();
    const float s = fold_row<ITERS>(r, lds, (size_t)row * nb, nb, j);
    if (j == 15 && row_raw < rows) y[row_raw] = s;
}

// ---- gate+up with GeGLU epilogue (model.rs:2093-2105, ops.rs:99-114) -------

template <int ITERS, int WAVES>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q4_0_geglu_kernel(const uint8_t *__restrict__ wg,
                                                                           const uint8_t *__restrict__ wu,
                                                                           const uint8_t *xpack,
                                                                           float *__restrict__ act, int rows,
                                                                           int nb)
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

    RowRegs<ITERS> rg, ru;
    load_row<ITERS>(rg, reinterpret_cast<const uint4 *>(wg), reinterpret_cast<const uint16_t *>(wg + nblk * 16),
                    (size_t)row * nb, nb, j);
    load_row<ITERS>(ru, reinterpret_cast<const uint4 *>(wu), reinterpret_cast<const uint16_t *>(wu + nblk * 16),
                    (size_t)row * nb, nb, j);
    __syncthreads();
    const float g = fold_row<ITERS>(rg, lds, (size_t)row * nb, nb, j);
    const float u = fold_row<ITERS>(ru, lds, (size_t)row * nb, nb, j);
    if (j == 15 && row_raw < rows) act[row_raw] = gelu_tanh(g) * u;
}

// ---- fused Q/K/V: y = [Wq x | Wk x | Wv x] (cuda.rs:2378-2404) -------------

template <int ITERS, int WAVES>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q4_0_qkv_kernel(const uint8_t *__restrict__ wq,
                                                                         const uint8_t *__restrict__ wk,
                                                                         const uint8_t *__restrict__ wv,
                                                                         const uint8_t *xpack,
                                                                         float *__restrict__ y, int q_rows,
                                                                         int kv_rows, int nb)
{
    extern __shared__ uint8_t lds[];
    if (threadIdx.x < 64) {
        stage_pack_wave(xpack, lds, nb);
        __syncthreads();
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int total = q_rows + 2 * kv_rows;
    const int quad = blockIdx.x * WAVES + (threadIdx.x >> 6) - 1;
    const int row_raw = quad * 4 + (lane >> 4);
    const int row = row_raw < total ? row_raw : total - 1;
    const uint8_t *w;
    int local, mrows;
    if (row < q_rows) { w = wq; local = row; mrows = q_rows; }
    else if (row < q_rows + kv_rows) { w = wk; local = row - q_rows; mrows = kv_rows; }
    else { w = wv; local = row - q_rows - kv_rows; mrows = kv_rows; }
    const size_t nblk = (size_t)mrows * nb;

    RowRegs<ITERS> r;
    load_row<ITERS>(r, reinterpret_cast<const uint4 *>(w), reinterpret_cast<const uint16_t *>(w + nblk * 16),
                    (size_t)local * nb, nb, j);
    __syncthreads();
    const float s = fold_row<ITERS>(r, lds, (size_t)local * nb, nb, j);
    if (j == 15 && row_raw < total) y[row_raw] = s;
}

// ---- raw GGUF layout --------------------------------------------------------
// The four rows of a wave are one contiguous span of 4*nb*18 bytes.  The
// wave copies the span into LDS with 16-byte loads when it is 16-byte
// aligned (nb % 8 == 0 and an aligned base), else with 2-byte loads, and
// reads each 18-byte block back from LDS.  One wave per workgroup.
template <int ITERS>
__global__ __launch_bounds__(64) void gemv_q4_0_gguf_kernel(const uint8_t *__restrict__ w,
                                                            const uint8_t *xpack,
                                                            float *__restrict__ y, int rows, int nb)
{
    extern __shared__ uint8_t lds[];
    uint8_t *act = lds;                                    // nb*40 bytes
    uint8_t *tile = lds + align_up((size_t)nb * 40, 16);   // 4 rows of raw blocks
    const int lane = threadIdx.x, j = lane & 15, rsub = lane >> 4;
    const int row0 = blockIdx.x * 4;
    const int nrows = rows - row0 < 4 ? rows - row0 : 4;
    const size_t row_bytes = (size_t)nb * 18;
    const uint8_t *span = w + (size_t)row0 * row_bytes;
    const size_t span_bytes = (size_t)nrows * row_bytes;
    if (((uintptr_t)span & 15u) == 0 && (span_bytes & 15u) == 0) {
        const uint4 *s = reinterpret_cast<const uint4 *>(span);
        uint4 *d = reinterpret_cast<uint4 *>(tile);
        for (size_t i = lane; i < span_bytes / 16; i += 64) d[i] = s[i];
    } else {
        const uint16_t *s = reinterpret_cast<const uint16_t *>(span);
        uint16_t *d = reinterpret_cast<uint16_t *>(tile);
        for (size_t i = lane; i < span_bytes / 2; i += 64) d[i] = s[i];
    }
    stage_pack_wave(xpack, act, nb);
    __syncthreads();
    const int row = rsub < nrows ? rsub : nrows - 1;
    const uint16_t *rowp = reinterpret_cast<const uint16_t *>(tile + (size_t)row * row_bytes);
    const int4 *aq = reinterpret_cast<const int4 *>(act);
    const float *ad = reinterpret_cast<const float *>(act + nb * 32);
    const int32_t *as = reinterpret_cast<const int32_t *>(act + nb * 36);
    float s = 0.0f;
    for (int it = 0; it < ITERS; ++it) {
        const int b = it * 16 + j;
        float t = 0.0f;
        if (b < nb) {
            const uint16_t *blk = rowp + b * 9;  // 18 bytes = 9 halfwords
            uint4 q;
            q.x = blk[1] | ((uint32_t)blk[2] << 16);
            q.y = blk[3] | ((uint32_t)blk[4] << 16);
            q.z = blk[5] | ((uint32_t)blk[6] << 16);
            q.w = blk[7] | ((uint32_t)blk[8] << 16);
            const int32_t isum = q4_0_isum(q, aq + 2 * b, as[b]);
            t = (float)isum * (f16_bits_to_f32(blk[0]) * ad[b]);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) s = fold16(s, t);
    }
    if (j == 15 && rsub < nrows) y[row0 + rsub] = s;
}

// ---- dispatch ---------------------------------------------------------------

// Waves per workgroup: enough rows per workgroup to amortise the LDS copy of
// the activation pack, few enough that the grid still covers all 256 CUs.
inline int waves_for(int rows) { return rows >= 8192 ? 4 : (rows >= 2048 ? 2 : 1); }

#define MRML_DISPATCH_ITERS(ITERS_VAL, BODY)                 \
    switch (ITERS_VAL) {                                     \
    case 1: { constexpr int IT = 1; BODY; } break;           \
    case 2: { constexpr int IT = 2; BODY; } break;           \
    case 3: { constexpr int IT = 3; BODY; } break;           \
    case 4: { constexpr int IT = 4; BODY; } break;           \
    case 5: { constexpr int IT = 5; BODY; } break;           \
    case 6: { constexpr int IT = 6; BODY; } break;           \
    case 8: { constexpr int IT = 8; BODY; } break;           \
    case 9: { constexpr int IT = 9; BODY; } break;           \
    case 12: { constexpr int IT = 12; BODY; } break;         \
    case 16: { constexpr int IT = 16; BODY; } break;         \
    case 18: { constexpr int IT = 18; BODY; } break;         \
    default: return fail(ctx, MRML_HIP_E_UNSUPPORTED,        \
                         "q4_0 matvec: cols=%d (%d blocks) has no kernel instance", nb * 32, nb); \
    }

#define MRML_DISPATCH_WAVES(WAVES_VAL, BODY)                 \
    switch (WAVES_VAL) {                                     \
    case 1: { constexpr int WV = 1; BODY; } break;           \
    case 2: { constexpr int WV = 2; BODY; } break;           \
    default: { constexpr int WV = 4; BODY; } break;          \
    }

}  // namespace

// The scale plane is read as 4-byte words, so the block count of each matrix
// (rows * cols/32) must be even: cols % 64 == 0 or an even row count.
static int check_even(mrml_hip_ctx *ctx, int32_t rows, int nb)
{
    if (((int64_t)rows * nb) & 1)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED,
                    "q4_0 matvec: rows*cols/32 = %lld is odd (needs cols %% 64 == 0 or even rows)",
                    (long long)rows * nb);
    return 0;
}

int launch_gemv_q4_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols)
{
    const int nb = cols / 32;
    if (int rc = check_even(ctx, rows, nb)) return rc;
    const int iters = (nb + 15) / 16;
    const int waves = waves_for(rows);
    const int quads = (rows + 3) / 4;
    const dim3 grid((quads + waves - 1) / waves);
    const size_t lds = act_pack_bytes(nb);
    MRML_DISPATCH_ITERS(iters, MRML_DISPATCH_WAVES(waves, {
        hipLaunchKernelGGL((gemv_q4_0_kernel<IT, WV>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,
                           (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb);
    }));
    return check_launch(ctx, "gemv_q4_0_kernel");
}

int launch_gemv_q4_0_geglu(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *xpack, float *act,
                           int32_t rows, int32_t cols)
{
    const int nb = cols / 32;
    if (int rc = check_even(ctx, rows, nb)) return rc;
    const int iters = (nb + 15) / 16;
    const int waves = waves_for(rows);
    const int quads = (rows + 3) / 4;
    const dim3 grid((quads + waves - 1) / waves);
    const size_t lds = act_pack_bytes(nb);
    MRML_DISPATCH_ITERS(iters, MRML_DISPATCH_WAVES(waves, {
        hipLaunchKernelGGL((gemv_q4_0_geglu_kernel<IT, WV>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,
                           (const uint8_t *)wg, (const uint8_t *)wu, (const uint8_t *)xpack, act, rows, nb);
    }));
    return check_launch(ctx, "gemv_q4_0_geglu_kernel");
}

int launch_gemv_q4_0_qkv(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const void *xpack,
                         float *y, int32_t q_rows, int32_t kv_rows, int32_t cols)
{
    const int nb = cols / 32;
    if (int rc = check_even(ctx, q_rows, nb)) return rc;
    if (int rc = check_even(ctx, kv_rows, nb)) return rc;
    const int iters = (nb + 15) / 16;
    const int total = q_rows + 2 * kv_rows;
    const int waves = waves_for(total);
    const int quads = (total + 3) / 4;
    const dim3 grid((quads + waves - 1) / waves);
    const size_t lds = act_pack_bytes(nb);
    MRML_DISPATCH_ITERS(iters, MRML_DISPATCH_WAVES(waves, {
        hipLaunchKernelGGL((gemv_q4_0_qkv_kernel<IT, WV>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,
                           (const uint8_t *)wq, (const uint8_t *)wk, (const uint8_t *)wv, (const uint8_t *)xpack,
                           y, q_rows, kv_rows, nb);
    }));
    return check_launch(ctx, "gemv_q4_0_qkv_kernel");
}

int launch_gemv_q4_0_gguf(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows,
                          int32_t cols)
{
    const int nb = cols / 32;
    const int iters = (nb + 15) / 16;
    const size_t lds = align_up((size_t)nb * 40, 16) + (size_t)4 * nb * 18;
    if (lds > 160 * 1024)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "gemv_q4_0_gguf: cols=%d needs %zu bytes of LDS", cols, lds);
    const dim3 grid((rows + 3) / 4);
    MRML_DISPATCH_ITERS(iters, {
        hipLaunchKernelGGL((gemv_q4_0_gguf_kernel<IT>), grid, dim3(64), lds, ctx->stream, (const uint8_t *)w,
                           (const uint8_t *)xpack, y, rows, nb);
    });
    return check_launch(ctx, "gemv_q4_0_gguf_kernel");
}

}  // namespace mrml
