// gemm_q4_0.hip -- batched Q4_0 x Q8_0 products (prefill, M tokens at once)
// with int8 MFMA on gfx950.
//
// Semantics (CudaDevice::gemm_q4_0, cuda.rs:2308-2332, layout x[token][cols],
// y[token][rows]; per token the CPU matvec of ops.rs:221-260):
//   isum_b(r, m) = sum_i (q_i(r) - 8) a_i(m)                   exact int32
//   y[m][r]      = (((0 + isum_0 (dw_0 da_0)) + isum_1 (dw_1 da_1)) + ...)
// block by block, each product and sum rounded separately, so every output
// is bit-identical to the batch-1 CPU path for that token.
//
// The integer part is one v_mfma_i32_32x32x32_i8 per (32 rows, 32 tokens,
// K block).  Lane l feeds row l%32 / token l%32 and K half l/32:
//   A = the row's 16 quant bytes, low nibbles (half 0) or high nibbles
//       (half 1), turned into signed bytes q-8 in registers (see sbytes), so
//       the MFMA result is isum itself;
//   B = the token's 16 int8 quants of that K half (the activation pack).
// Lane l receives D[8j+4(l/32)+i][l%32] in element 4j+i: 16 rows of ONE
// token, so the token's block scale is a per-lane scalar and the rows'
// scales come from LDS as float4s.
//
// The ordered f32 fold runs on the VALU: 4 instructions per output per block
// (cvt, dw*da, *, +) against one MFMA per 1024 outputs, so the kernel is
// VALU-bound by construction.  Everything else is arranged around keeping the
// VALU busy: the row tile's scales are staged once in LDS, operand loads run
// kPF blocks ahead (buffer loads, which the compiler keeps where they are
// written), and each block's MFMA is issued before the previous block is
// folded so its latency overlaps VALU work.

#include "device.h"
#include "internal.h"

namespace mrml {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmWaves = 4;             // 32-token tiles per workgroup, sharing one 32-row tile
constexpr int kPF = 4;                    // operand prefetch distance, blocks
constexpr int kBufferFlags = 0x00020000;  // buffer resource word 3 (raw 32-bit data) on gfx9

struct Operands {
    u32x4 w;   // the row's 16 quant bytes
    u32x4 a;   // the token's 16 quants of this K half
    float da;  // the token's block scale
};

// Four nibbles per dword (selected by shift 0 or 4) -> four signed bytes q-8.
// Per byte: (q | 0x80) - 8 stays within 0x78..0x87, so no borrow crosses a
// byte; flipping bit 7 then gives q-8 modulo 256.
__device__ __forceinline__ int sbytes(uint32_t v, int sh)
{
    const uint32_t n = ((v >> sh) & 0x0F0F0F0Fu) | 0x80808080u;
    return (int)((n - 0x08080808u) ^ 0x80808080u);
}

__global__ __launch_bounds__(64 * kGemmWaves) void gemm_q4_0_mfma_kernel(const uint8_t *__restrict__ w,
                                                                         const uint8_t *__restrict__ xpack,
                                                                         float *__restrict__ y, int rows, int nb,
                                                                         int batch)
{
    extern __shared__ __align__(16) float dws[];  // [nb][32]: the row tile's block scales, f32
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * 32;
    const uint32_t qs_bytes = (uint32_t)rows * nb * 16;

    // The 32 rows' scales are one contiguous run of 32*nb f16 in the scale
    // plane (64*nb bytes, 16-byte aligned): 8 per 16-byte load, up to kSL
    // loads of a thread in flight together.
    {
        constexpr int kSL = 4, kStride = 64 * kGemmWaves;
        const u32x4 *src = reinterpret_cast<const u32x4 *>(w + qs_bytes) + (size_t)r0 * nb / 8;
        for (int i0 = 0; i0 < 4 * nb; i0 += kSL * kStride) {
            u32x4 v[kSL];
#pragma unroll
            for (int k = 0; k < kSL; ++k) {
                const int i = i0 + tid + k * kStride;
                if (i < 4 * nb) v[k] = src[i];
            }
#pragma unroll
            for (int k = 0; k < kSL; ++k) {
                const int i = i0 + tid + k * kStride;
                if (i >= 4 * nb) break;
                int r = 8 * i / nb, b = 8 * i - r * nb;  // element 8i = row r, block b
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    dws[b * 32 + r] = f16_bits_to_f32((v[k][j >> 1] >> (16 * (j & 1))) & 0xffffu);
                    if (++b == nb) b = 0, ++r;
                }
            }
        }
    }
    __syncthreads();
    const int t0 = (blockIdx.y * kGemmWaves + wave) * 32;
    if (t0 >= batch) return;  // no barrier follows
    const int tl = lane & 31, h = lane >> 5;
    const int tok = t0 + tl < batch ? t0 + tl : batch - 1;  // tail lanes recompute the last token
    const uint32_t ntot = (uint32_t)batch * nb;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void *)w, (short)0, (int)qs_bytes,
                                                                        kBufferFlags);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)xpack, (short)0, (int)(ntot * 36),
                                                                        kBufferFlags);
    const uint32_t wo = (uint32_t)(r0 + tl) * nb * 16;
    const uint32_t ao = (uint32_t)tok * nb * 32 + 16 * h;
    const uint32_t so = ntot * 32 + (uint32_t)tok * nb * 4;
    const int sh = 4 * h;

    // Loads past the lane's last block read neighbouring rows / tokens or,
    // past the end of a buffer, zeros (buffer range check); never used.
    auto load = [&](int b, Operands &o) {
        o.w = __builtin_amdgcn_raw_buffer_load_b128(wr, wo + 16u * b, 0, 0);
        o.a = __builtin_amdgcn_raw_buffer_load_b128(xr, ao + 32u * b, 0, 0);
        o.da = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, so + 4u * b, 0, 0));
    };
    auto mfma = [&](const Operands &o) {
        const v4i a = {sbytes(o.w.x, sh), sbytes(o.w.y, sh), sbytes(o.w.z, sh), sbytes(o.w.w, sh)};
        const v4i bq = {(int)o.a.x, (int)o.a.y, (int)o.a.z, (int)o.a.w};
        const v16i zero = {};
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, zero, 0, 0, 0);
    };

    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
    // Block b's fold: the four float4s of row scales are read from LDS first
    // (one wait for all four), then 16 x (cvt, dw*da, *, +) in block order.
    auto fold = [&](const v16i &d, float da, int b) {
        const float4 *dwb = reinterpret_cast<const float4 *>(dws + b * 32 + 4 * h);
        float4 dw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) dw[j] = dwb[2 * j];  // rows 8j + 4h + 0..3
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float dwv[4] = {dw[j].x, dw[j].y, dw[j].z, dw[j].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[4 * j + i] = acc[4 * j + i] + (float)d[4 * j + i] * (dwv[i] * da);
        }
    };

    // ring[s] holds the operands of block b with b % kPF == s.  Step b:
    // issue block b+1's MFMA, fold block b (its MFMA result from the previous
    // step, its token scale still in its slot), then refill block b's slot
    // with block b+kPF.  Scheduling barriers keep that order (the scheduler
    // would otherwise gather the loads at the end of the loop and wait for
    // all of them at its top), so each wait covers only the loads of the
    // block about to be used.  The main loop has no branches; it may issue
    // the MFMA and loads of blocks >= nb, whose results are never folded.
    Operands ring[kPF];
#pragma unroll
    for (int s = 0; s < kPF; ++s) load(s, ring[s]);
    v16i d = mfma(ring[0]);
    auto step = [&](int b, Operands &cur, const Operands &next, bool refill) {
        const v16i dn = mfma(next);
        __builtin_amdgcn_sched_barrier(0);
        fold(d, cur.da, b);
        __builtin_amdgcn_sched_barrier(0);
        if (refill) load(b + kPF, cur);
        d = dn;
    };
    int b0 = 0;
    for (; b0 + kPF <= nb; b0 += kPF) {
#pragma unroll
        for (int s = 0; s < kPF; ++s) step(b0 + s, ring[s], ring[(s + 1) % kPF], true);
    }
#pragma unroll
    for (int s = 0; s < kPF - 1; ++s)  // the last nb % kPF blocks
        if (b0 + s < nb) step(b0 + s, ring[s], ring[(s + 1) % kPF], false);
    if (t0 + tl < batch) {
        float *yr = y + (size_t)(t0 + tl) * rows + r0 + 4 * h;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<float4 *>(yr + 8 * j) = make_float4(acc[4 * j], acc[4 * j + 1], acc[4 * j + 2],
                                                                  acc[4 * j + 3]);
    }
}

}  // namespace

bool gemm_shape_ok(int32_t rows, int32_t cols, int32_t batch)
{
    if (rows <= 0 || rows % 32 != 0 || cols <= 0 || cols % 32 != 0 || cols / 32 > 512 || batch <= 0) return false;
    // 32-bit buffer offsets: the quant plane of W and the whole activation pack
    const int64_t nb = cols / 32;
    return (int64_t)rows * nb * 16 < INT32_MAX && (int64_t)batch * nb * 40 < INT32_MAX;
}

int launch_gemm_q4_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols,
                     int32_t batch)
{
    const int nb = cols / 32;
    const dim3 grid(rows / 32, (batch + 32 * kGemmWaves - 1) / (32 * kGemmWaves));
    hipLaunchKernelGGL(gemm_q4_0_mfma_kernel, grid, dim3(64 * kGemmWaves), (size_t)nb * 32 * sizeof(float),
                       ctx->stream, (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb, batch);
    return check_launch(ctx, "gemm_q4_0_mfma_kernel");
}

}  // namespace mrml
