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
// K block) -- or, for the last row tiles of a product whose tiles number just
// over one per SIMD, two v_mfma_i32_16x16x32_i8 per (32 rows, 16 tokens, K
// block) (gemm_tile below).  Lane l feeds row l%32 / token l%32 and K half l/32:
//   A = the row's 16 quant bytes, low nibbles (half 0) or high nibbles
//       (half 1), as signed bytes q-8 (see sbytes, applied when the weights
//       are staged), so the MFMA result is isum itself;
//   B = the token's 16 int8 quants of that K half.
// Lane l receives D[8j+4(l/32)+i][l%32] in element 4j+i: 16 rows of ONE
// token, so the token's block scale is a per-lane scalar and the rows'
// scales are float4 broadcasts from LDS.
//
// The ordered f32 fold runs on the VALU: 4 instructions per output per block
// (3 with RELAXED, the tolerance path's one-FMA fold)
// against one MFMA per 1024 outputs.  Measured on gfx950: an MFMA holds its
// SIMD's VALU issue while it executes (about 36 cycles for this one); f32
// mul/add and integer ALU ops issue from two waves at once (about 2.4 SIMD
// cycles each) while v_cvt_f32_i32 does not (about 4.5).  So the int->float
// conversion is done without it: the MFMA accumulates onto C = 0x4B400000,
// the bits of 1.5*2^23, and since |isum| <= 32*8*128 < 2^22 the sum stays in
// the binade [2^23, 2^24) where one unit of the bit pattern is one unit of
// value: D reinterpreted as f32 is exactly 1.5*2^23 + isum, and one exact
// subtraction returns (float)isum.  Per output per block: sub, dw*da, *, +.
// (The scale products form a rank-1 matrix that a v_mfma_f32_32x32x2_f32
// could produce, but that MFMA costs more SIMD time than the 16 multiplies it
// replaces.)  Operand feed:
//   - B comes from a GEMM pack written in MFMA lane order (one 1 KB run of
//     quants and one 128-byte run of scales per 32 tokens and block), read
//     with one coalesced load each, kPF blocks ahead of use;
//   - A is shared by the workgroup's four waves (four 32-token groups, or
//     four 16-token halves, over one 32-row tile): kKC-block chunks of the
//     32 rows (128 contiguous bytes
//     per row) and their f16 scales are loaded with coalesced loads into
//     registers one chunk ahead, turned into signed bytes once (both K
//     halves) and staged through kNBuf LDS buffers, one barrier per chunk.

#include <mutex>

#include "device.h"
#include "internal.h"

namespace mrml {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmWaves = 4;             // 32-token groups per workgroup, sharing one 32-row tile
constexpr int kPF = 4;                    // B prefetch distance, blocks
constexpr int kKC = 8;                    // blocks per A chunk
constexpr int kNBuf = 3;                  // A chunk buffers in LDS
constexpr int kBufferFlags = 0x00020000;  // buffer resource word 3 (raw 32-bit data) on gfx9
constexpr float kMagic = 12582912.0f;      // 1.5 * 2^23
constexpr int kMagicBits = 0x4B400000;     // its f32 bit pattern
constexpr int kSIMDs = 1024;               // MI355X: 256 CUs x 4 SIMDs

// quant.rs:193-228 per block (q8_0_block8x4), written as a GEMM pack.  One
// workgroup per (group, block): thread 8t+l handles token 32g+t, values
// 4l..4l+3 of block b.  Tokens past `batch` are written as zeros.  GEGLU:
// the values quantized are gelu_tanh(x) * u elementwise (the GeGLU epilogue
// of the matvec kernels, model.rs:2093-2105), formed in registers, so the
// down projection's pack comes straight from the gate and up products.
// Token m's values start at x + m*ld4*4 (and u + m*ld4*4).
template <bool GEGLU>
__global__ __launch_bounds__(256) void quantize_gemm_pack_kernel(const float *__restrict__ x,
                                                                 const float *__restrict__ u,
                                                                 uint8_t *__restrict__ gp, int nb, int batch,
                                                                 int ngroups, int ld4)
{
    const int g = blockIdx.x / nb, b = blockIdx.x - g * nb;
    const int t = threadIdx.x >> 3, l = threadIdx.x & 7, m = 32 * g + t;
    const int ms = m < batch ? m : batch - 1;  // every lane takes part in the block reductions
    uint32_t dbits;
    int s;
    const size_t i4 = (size_t)ms * ld4 + b * 8 + l;
    float4 v = reinterpret_cast<const float4 *>(x)[i4];
    if constexpr (GEGLU) {
        const float4 w = reinterpret_cast<const float4 *>(u)[i4];
        v.x = gelu_tanh(v.x) * w.x;
        v.y = gelu_tanh(v.y) * w.y;
        v.z = gelu_tanh(v.z) * w.z;
        v.w = gelu_tanh(v.w) * w.w;
    }
    const uint32_t q = q8_0_block8x4(v, dbits, s);
    const bool real = m < batch;
    gemm_pack_put(gp, ngroups, nb, m, b, l, real ? q : 0u, real ? f16_bits_to_f32(dbits) : 0.0f);
}

// An activation pack of batch*nb blocks (block (m,b) at m*nb+b) -> GEMM pack.
__global__ __launch_bounds__(256) void gemm_pack_from_act_kernel(const uint8_t *__restrict__ pack,
                                                                 uint8_t *__restrict__ gp, int nb, int batch,
                                                                 int ngroups)
{
    const int g = blockIdx.x / nb, b = blockIdx.x - g * nb;
    const int t = threadIdx.x >> 3, l = threadIdx.x & 7, m = 32 * g + t;
    uint32_t q = 0;
    float d = 0.0f;
    if (m < batch) {
        const size_t blk = (size_t)m * nb + b;
        q = reinterpret_cast<const uint32_t *>(pack)[blk * 8 + l];
        d = reinterpret_cast<const float *>(pack + (size_t)batch * nb * 32)[blk];
    }
    gemm_pack_put(gp, ngroups, nb, m, b, l, q, d);
}

// Four nibbles per dword (selected by shift 0 or 4) -> four signed bytes q-8.
// Per byte: (q | 0x80) - 8 stays within 0x78..0x87, so no borrow crosses a
// byte; flipping bit 7 then gives q-8 modulo 256.
__device__ __forceinline__ int sbytes(uint32_t v, int sh)
{
    const uint32_t n = ((v >> sh) & 0x0F0F0F0Fu) | 0x80808080u;
    return (int)((n - 0x08080808u) ^ 0x80808080u);
}

// LDS writes of this wave complete, then the workgroup barrier.  As inline
// asm with a memory clobber, no LDS access is moved across it; outstanding
// global loads (the operand prefetch) stay in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Up to three weight matrices stacked by rows (q|k|v) for one launch: row
// tile rt (32 rows) of the stack belongs to the matrix whose row range holds
// it (every matrix but the last a multiple of 32 rows), and its outputs go
// to the stacked output column r (y rows hold the stack).
constexpr int kGemmMaxMats = 3;
struct GemmMats {
    const uint8_t *w[kGemmMaxMats];
    int rows[kGemmMaxMats];
    int n;
};

struct BOps {
    u32x4 a;   // the token's 16 quants of this K half
    float da;  // the token's block scale
};

// RELAXED: each block term joins its output's sum with one FMA instead of
// a product and a separate add (the integer sums stay exact; the f32 sums
// round once per block instead of twice) -- the tolerance path's prefill.
//
// Tile of one wave over all of K:
//   FULL: 32 rows x 32 tokens, one v_mfma_i32_32x32x32_i8 a block (lane l:
//         row / token l%32, K half l/32; 16 outputs a lane, rows
//         8j + 4(l/32) + i of token l%32);
//   HALF: 32 rows x 16 tokens (half of a token group), two
//         v_mfma_i32_16x16x32_i8 a block, rows 0..15 and 16..31 (lane l:
//         row / token l%16, K bytes 8(l/16)..+8; 8 outputs a lane, rows
//         16j + 4(l/16) + i of token l%16).
// A HALF wave folds half the outputs of a FULL one for the same operand
// reads, so it serves only to spread a product whose FULL tiles number just
// over one per SIMD (the launch below).
template <bool RELAXED, bool HALF>
__device__ __forceinline__ void gemm_tile(const GemmMats &mats, const uint8_t *__restrict__ gp,
                                          float *__restrict__ y, int rows, int nb, int batch, int ngroups, int ldy,
                                          int vec, int rt, int gsel, u32x4 (&sa)[kNBuf][kKC][2][32],
                                          float (&sdw)[kNBuf][kKC][32])
{
    constexpr int NACC = HALF ? 8 : 16;  // outputs a lane
    const int tid = threadIdx.x, lane = tid & 63;
    const int r0 = rt * 32;
    // FULL: token group gsel; HALF: half gsel & 1 of token group gsel >> 1.
    // A group >= ngroups computes on zeros and stores nothing.
    const int g = HALF ? gsel >> 1 : gsel;
    const int tl = HALF ? 16 * (gsel & 1) + (lane & 15) : lane & 31;  // the lane's token in its group
    const int q = lane >> 4, h = lane >> 5;                            // HALF: K quarter; FULL: K half
    const int rbase = HALF ? 4 * q : 4 * h;                           // first row of the lane's outputs
    constexpr int rstep = HALF ? 16 : 8;                              // rows between its output quads
    // the tile's matrix (uniform): local rows r0 - mbase of mrows
    int m = 0, mbase = 0;
    while (m + 1 < mats.n && r0 >= mbase + mats.rows[m]) mbase += mats.rows[m++];
    const int mrows = mats.rows[m], r0l = r0 - mbase;
    const uint32_t qs_bytes = (uint32_t)mrows * nb * 16;
    // Loads past a row's last block read the next row or, past the end of a
    // buffer, zeros (buffer range check); such blocks are never folded.
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void *)mats.w[m], (short)0,
                                                                        (int)(qs_bytes + (uint32_t)mrows * nb * 2),
                                                                        kBufferFlags);
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)gp, (short)0, (int)((uint32_t)ngroups * nb * 1152), kBufferFlags);

    // A chunk c: thread (row ar, block ak) loads 16 quant bytes and one f16 scale.
    const int ar = tid >> 3, ak = tid & 7;
    const uint32_t a_off = ((uint32_t)(r0l + ar) * nb + ak) * 16;
    const uint32_t s_off = qs_bytes + ((uint32_t)(r0l + ar) * nb + ak) * 2;
    u32x4 areg;
    uint32_t sreg;
    auto load_chunk = [&](int c) {
        areg = __builtin_amdgcn_raw_buffer_load_b128(wr, a_off + (uint32_t)c * (kKC * 16), 0, 0);
        sreg = __builtin_amdgcn_raw_buffer_load_b16(wr, s_off + (uint32_t)c * (kKC * 2), 0, 0);
    };
    auto store_chunk = [&](int buf) {
        sa[buf][ak][0][ar] = u32x4{(uint32_t)sbytes(areg.x, 0), (uint32_t)sbytes(areg.y, 0),
                                   (uint32_t)sbytes(areg.z, 0), (uint32_t)sbytes(areg.w, 0)};
        sa[buf][ak][1][ar] = u32x4{(uint32_t)sbytes(areg.x, 4), (uint32_t)sbytes(areg.y, 4),
                                   (uint32_t)sbytes(areg.z, 4), (uint32_t)sbytes(areg.w, 4)};
        sdw[buf][ak][ar] = f16_bits_to_f32(sreg);
    };

    // B: the lane's quants of its token (FULL: 16 bytes, its K half; HALF:
    // 8 bytes, its K quarter) and the token's block scale.
    const uint32_t b_off = HALF ? ((uint32_t)g * nb * 64 + 32 * (q >> 1) + tl) * 16 + 8 * (q & 1)
                                : ((uint32_t)g * nb * 64 + lane) * 16;
    const uint32_t d_off = (uint32_t)ngroups * nb * 1024 + ((uint32_t)g * nb * 32 + tl) * 4;
    auto load_b = [&](int b, BOps &o) {
        if constexpr (HALF) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(gr, b_off + (uint32_t)b * 1024, 0, 0);
            o.a = u32x4{v[0], v[1], 0u, 0u};
        } else {
            o.a = __builtin_amdgcn_raw_buffer_load_b128(gr, b_off + (uint32_t)b * 1024, 0, 0);
        }
        o.da = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(gr, d_off + (uint32_t)b * 128, 0, 0));
    };
    // The lane's A operand of a block (HALF: rows l%16 and 16 + l%16, 8 bytes each).
    auto read_a = [&](int buf, int kc) {
        if constexpr (HALF) {
            const uint2 a0 = reinterpret_cast<const uint2 *>(&sa[buf][kc][q >> 1][lane & 15])[q & 1];
            const uint2 a1 = reinterpret_cast<const uint2 *>(&sa[buf][kc][q >> 1][16 + (lane & 15)])[q & 1];
            return u32x4{a0.x, a0.y, a1.x, a1.y};
        } else {
            return sa[buf][kc][h][tl];
        }
    };
    // C of every MFMA: the f32 bits of kMagic (see the header).
    auto mfma = [&](const u32x4 wv, const BOps &o) {
        v16i d;
        if constexpr (HALF) {
            const v4i cm = {kMagicBits, kMagicBits, kMagicBits, kMagicBits};
            const long bq = (long)((uint64_t)o.a.x | ((uint64_t)o.a.y << 32));
            const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)((uint64_t)wv.x | ((uint64_t)wv.y << 32)), bq,
                                                                 cm, 0, 0, 0);
            const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)((uint64_t)wv.z | ((uint64_t)wv.w << 32)), bq,
                                                                 cm, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                d[e] = d0[e];
                d[4 + e] = d1[e];
                d[8 + e] = 0;
                d[12 + e] = 0;
            }
        } else {
            v16i cmagic;
#pragma unroll
            for (int e = 0; e < 16; ++e) cmagic[e] = kMagicBits;
            const v4i a = {(int)wv.x, (int)wv.y, (int)wv.z, (int)wv.w};
            const v4i bq = {(int)o.a.x, (int)o.a.y, (int)o.a.z, (int)o.a.w};
            d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, cmagic, 0, 0, 0);
        }
        return d;
    };

    float acc[NACC];
#pragma unroll
    for (int e = 0; e < NACC; ++e) acc[e] = 0.0f;
    // The lane's row scales of a block: NACC/4 float4s, rows rstep*j + rbase + 0..3.
    auto read_dw = [&](int buf, int kc, float4 (&dw)[4]) {
        const float4 *dwb = reinterpret_cast<const float4 *>(&sdw[buf][kc][rbase]);
#pragma unroll
        for (int j = 0; j < NACC / 4; ++j) dw[j] = dwb[(rstep / 4) * j];
    };
    // Block fold: NACC x (isum, dw*da, *, +).
    auto fold = [&](const v16i &d, float da, const float4 (&dw)[4]) {
#pragma unroll
        for (int j = 0; j < NACC / 4; ++j) {
            const float dwv[4] = {dw[j].x, dw[j].y, dw[j].z, dw[j].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // (the element is copied out first: bit_cast of an ext-vector
                // element lvalue reads element 0 in this compiler)
                const int de = d[4 * j + i];
                const float isum = __builtin_bit_cast(float, de) - kMagic;  // exact
                if constexpr (RELAXED) acc[4 * j + i] = __builtin_fmaf(isum, dwv[i] * da, acc[4 * j + i]);
                else acc[4 * j + i] = acc[4 * j + i] + isum * (dwv[i] * da);
            }
        }
    };

    // Chunks 0 and 1 into LDS, chunk 2 in flight; B blocks 0..kPF-1 in flight.
    load_chunk(0);
    store_chunk(0);
    load_chunk(1);
    store_chunk(1);
    lds_barrier();
    load_chunk(2);
    BOps ring[kPF];
#pragma unroll
    for (int s = 0; s < kPF; ++s) load_b(s, ring[s]);

    // Step (block b = kKC*c + kc), software-pipelined so that no LDS read or
    // MFMA result is waited for right after it is issued:
    //   - the MFMA of block b+1, on the A operand read at step b-1;
    //   - the LDS reads of block b+2's A operand and block b+1's row scales
    //     (from the next chunk's buffer, already whole, near a chunk's end);
    //   - the fold of block b (result and row scales from step b-1);
    //   - block b+kPF into block b's B slot.
    // A wave alone on its SIMD (down: 1152 tiles for 1024 SIMDs) otherwise
    // waits out each latency every block: down 75.3 -> 71.1 us, gate and up
    // about 1.5 us each.  Past the last block these MFMAs and reads work on
    // in-range leftovers and are never folded.  A scheduling barrier keeps the
    // refill after the fold (the scheduler would otherwise gather the loads
    // and wait for them all at once), so each wait covers only the block about
    // to be used.  Loads of blocks >= nb are never used.
    // Chunk reuse: at the end of chunk c, chunk c+2 is written into buffer
    // (c+2)%3 = (c-1)%3, whose readers (chunk c-1's reads and MFMAs, the
    // first of them issued during chunk c-2, and its folds) all come before
    // the barrier that ended chunk c-1.
    int c = 0, cb = 0, nbf = 1, wb = 2;  // chunk, its buffer, the next chunk's buffer, the buffer to write
    v16i dq = mfma(read_a(cb, 0), ring[0]);
    u32x4 an = read_a(cb, 1);  // block 1 (kKC > 1)
    float4 dwc[4];
    read_dw(cb, 0, dwc);
    auto step = [&](int kc, int nbuf, int nkc, int nbuf2, int nkc2, bool refill, int b) {
        const v16i dn = mfma(an, ring[(kc + 1) % kPF]);
        an = read_a(nbuf2, nkc2);
        float4 dwn[4];
        read_dw(nbuf, nkc, dwn);
        fold(dq, ring[kc % kPF].da, dwc);
        __builtin_amdgcn_sched_barrier(0);
        if (refill) load_b(b + kPF, ring[kc % kPF]);
        dq = dn;
#pragma unroll
        for (int j = 0; j < NACC / 4; ++j) dwc[j] = dwn[j];
    };
    static_assert(kKC > 2, "blocks b+1 and b+2 are each in this chunk or the next");
    for (; (c + 1) * kKC <= nb; ++c) {
#pragma unroll
        for (int kc = 0; kc < kKC; ++kc)
            step(kc, kc + 1 < kKC ? cb : nbf, (kc + 1) % kKC, kc + 2 < kKC ? cb : nbf, (kc + 2) % kKC, true,
                 c * kKC + kc);
        store_chunk(wb);
        lds_barrier();
        load_chunk(c + 3);
        cb = nbf;
        nbf = wb;
        wb = wb == kNBuf - 1 ? 0 : wb + 1;
    }
    // The last nb % kKC blocks.  Their ring slots are refilled as in a full
    // chunk: with more than kPF of them, blocks kPF.. reuse the slots of
    // blocks 0.. (loads of blocks >= nb are in range of the buffer or read
    // zeros, and are never folded).
#pragma unroll
    for (int kc = 0; kc < kKC - 1; ++kc)
        if (c * kKC + kc < nb) step(kc, cb, kc + 1, cb, (kc + 2) % kKC, kc + kPF < kKC - 1, c * kKC + kc);

    const int tok = g * 32 + tl;
    if (tok < batch) {
        float *yr = y + (size_t)tok * ldy + r0 + rbase;  // row stride ldy (rows when packed)
        if (r0 + 32 <= rows && vec) {
#pragma unroll
            for (int j = 0; j < NACC / 4; ++j)
                *reinterpret_cast<float4 *>(yr + rstep * j) = make_float4(acc[4 * j], acc[4 * j + 1],
                                                                          acc[4 * j + 2], acc[4 * j + 3]);
        } else {
            // the last tile of a row count that is not a multiple of 32, or
            // an output that float4 stores cannot reach (a stride that is
            // not a multiple of 4, or y not 16-byte aligned): one float each
            // for the rows that exist (rows past them are computed on
            // whatever their loads read, and never stored)
#pragma unroll
            for (int j = 0; j < NACC / 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (r0 + rbase + rstep * j + i < rows) yr[rstep * j + i] = acc[4 * j + i];
        }
    }
}

// Row tiles [0, rt_full) in FULL waves (workgroup: one row tile, four token
// groups), the rest in HALF waves (workgroup: one row tile, four half
// groups); the workgroup index picks the form, so every wave of a
// workgroup takes the same one.
template <bool RELAXED>
__global__ __launch_bounds__(64 * kGemmWaves) void gemm_q4_0_mfma_kernel(const GemmMats mats,
                                                                         const uint8_t *__restrict__ gp,
                                                                         float *__restrict__ y, int rows, int nb,
                                                                         int batch, int ngroups, int ldy, int vec,
                                                                         int rt_full)
{
    __shared__ __align__(16) u32x4 sa[kNBuf][kKC][2][32];  // A chunks: [block][K half][row] 16 signed bytes
    __shared__ __align__(16) float sdw[kNBuf][kKC][32];  // their row scales, f32
    const int wave = threadIdx.x >> 6, wg = blockIdx.x;
    const int nfull = rt_full * ((ngroups + kGemmWaves - 1) / kGemmWaves);
    if (wg < nfull) {
        gemm_tile<RELAXED, false>(mats, gp, y, rows, nb, batch, ngroups, ldy, vec, wg % rt_full,
                                  (wg / rt_full) * kGemmWaves + wave, sa, sdw);
    } else {
        const int rt_half = (rows + 31) / 32 - rt_full, hw = wg - nfull;
        gemm_tile<RELAXED, true>(mats, gp, y, rows, nb, batch, ngroups, ldy, vec, rt_full + hw % rt_half,
                                 (hw / rt_half) * kGemmWaves + wave, sa, sdw);
    }
}

// Device scratch of the allocation-free GEMM entry point
// (mrml_hip_gemm_q4_0_noalloc): the GEMM pack of its activations lives in
// this file-scope array, one copy per GPU, held until the process ends.  Host
// code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): gemm_noalloc_scratch() resolves each
// device's address once, with hipGetSymbolAddress, and launches take that.
// Every call on a GPU shares its copy, so calls that overlap on one GPU race.
// Each call writes the whole pack it reads (tokens past the batch as zeros),
// so nothing has to start zeroed.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) uint8_t gemm_noalloc_scratch_buf[kNoAllocScratchBytes];

}  // namespace

size_t gemm_noalloc_scratch_bytes() { return kNoAllocScratchBytes; }

int gemm_noalloc_scratch(mrml_hip_ctx *ctx, void **out)
{
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void *addr[kMaxDevices];
    *out = nullptr;
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "gemm scratch: device index %d above %d", ctx->device, kMaxDevices);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[ctx->device]) {
        // The context's device is current (every entry point makes it so).
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(gemm_noalloc_scratch_buf));
        if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress (gemm scratch)");
        if (!p) return fail(ctx, MRML_HIP_E_HIP, "hipGetSymbolAddress (gemm scratch) returned null");
        addr[ctx->device] = p;
    }
    *out = addr[ctx->device];
    return MRML_HIP_OK;
}

bool gemm_shape_ok(int32_t rows, int32_t cols, int32_t batch)
{
    if (rows <= 0 || cols <= 0 || cols % 32 != 0 || batch <= 0) return false;
    // 32-bit buffer offsets: the whole of W and of the GEMM pack
    const int64_t nb = cols / 32;
    return (int64_t)rows * nb * 18 < INT32_MAX && ((int64_t)batch + 31) / 32 * nb * 1152 < INT32_MAX &&
           (int64_t)batch * nb * 40 < INT32_MAX;
}

size_t gemm_pack_bytes(int32_t cols, int32_t batch) { return (size_t)gemm_groups(batch) * (cols / 32) * 1152; }

int launch_gemm_pack_quantize(mrml_hip_ctx *ctx, const float *x, void *gpack, int32_t cols, int32_t batch)
{
    const int nb = cols / 32, ng = gemm_groups(batch);
    hipLaunchKernelGGL(quantize_gemm_pack_kernel<false>, dim3((unsigned)(ng * nb)), dim3(256), 0, ctx->stream, x,
                       nullptr, (uint8_t *)gpack, nb, batch, ng, nb * 8);
    return check_launch(ctx, "quantize_gemm_pack_kernel");
}

int launch_gemm_pack_geglu(mrml_hip_ctx *ctx, const float *g, const float *u, int32_t ld, void *gpack,
                           int32_t cols, int32_t batch)
{
    const int nb = cols / 32, ng = gemm_groups(batch);
    if (ld % 4 != 0 || ld < cols || ((uintptr_t)g | (uintptr_t)u) % 16 != 0)
        return fail(ctx, MRML_HIP_E_INVALID, "gemm pack (geglu): row stride %d or operands not 16-byte aligned", ld);
    hipLaunchKernelGGL(quantize_gemm_pack_kernel<true>, dim3((unsigned)(ng * nb)), dim3(256), 0, ctx->stream, g, u,
                       (uint8_t *)gpack, nb, batch, ng, ld / 4);
    return check_launch(ctx, "quantize_gemm_pack_kernel<geglu>");
}

int launch_gemm_pack_from_act(mrml_hip_ctx *ctx, const void *pack, void *gpack, int32_t cols, int32_t batch)
{
    const int nb = cols / 32, ng = gemm_groups(batch);
    hipLaunchKernelGGL(gemm_pack_from_act_kernel, dim3((unsigned)(ng * nb)), dim3(256), 0, ctx->stream,
                       (const uint8_t *)pack, (uint8_t *)gpack, nb, batch, ng);
    return check_launch(ctx, "gemm_pack_from_act_kernel");
}

static int launch_gemm_mats(mrml_hip_ctx *ctx, const GemmMats &mats, const void *gpack, float *y, int32_t rows,
                            int32_t cols, int32_t batch, int32_t ldy, bool relaxed)
{
    const int nb = cols / 32, ng = gemm_groups(batch);
    if (ldy == 0) ldy = rows;
    if (ldy < rows || ((uintptr_t)y & 3) != 0)
        return fail(ctx, MRML_HIP_E_INVALID, "gemm_q4_0: output stride %d below rows %d, or y not 4-byte aligned",
                    ldy, rows);
    const int vec = (ldy % 4 == 0 && ((uintptr_t)y & 15) == 0) ? 1 : 0;  // float4 stores reach every output row
    // FULL waves, one per (row tile, token group).  When they number just
    // over one per SIMD (down at M = 512: 1152 for 1024), the SIMDs holding
    // two of them set the launch's time; then only as many row tiles as
    // give every SIMD one FULL wave stay FULL and the rest run as HALF waves
    // (two per token group), which add a little over half a wave's work to
    // some SIMDs instead of a whole one.
    const int rt = (rows + 31) / 32, gq = (ng + kGemmWaves - 1) / kGemmWaves;
    const int full_waves = rt * gq * kGemmWaves;
    int rt_full = rt;
    if (full_waves > kSIMDs && 2 * full_waves <= 3 * kSIMDs) rt_full = kSIMDs / (gq * kGemmWaves);
    const int hq = (2 * ng + kGemmWaves - 1) / kGemmWaves;  // workgroups of HALF waves per row tile
    const dim3 grid((unsigned)(rt_full * gq + (rt - rt_full) * hq));
    if (relaxed)
        hipLaunchKernelGGL(gemm_q4_0_mfma_kernel<true>, grid, dim3(64 * kGemmWaves), 0, ctx->stream, mats,
                           (const uint8_t *)gpack, y, rows, nb, batch, ng, ldy, vec, rt_full);
    else
        hipLaunchKernelGGL(gemm_q4_0_mfma_kernel<false>, grid, dim3(64 * kGemmWaves), 0, ctx->stream, mats,
                           (const uint8_t *)gpack, y, rows, nb, batch, ng, ldy, vec, rt_full);
    return check_launch(ctx, "gemm_q4_0_mfma_kernel");
}

int launch_gemm_q4_0(mrml_hip_ctx *ctx, const void *w, const void *gpack, float *y, int32_t rows, int32_t cols,
                     int32_t batch, int32_t ldy, bool relaxed)
{
    GemmMats mats{};
    mats.w[0] = (const uint8_t *)w;
    mats.rows[0] = rows;
    mats.n = 1;
    return launch_gemm_mats(ctx, mats, gpack, y, rows, cols, batch, ldy, relaxed);
}

// Up to three products over one GEMM pack in one launch, their outputs
// stacked along y's rows (matrix m's rows start after those of the earlier
// ones): every matrix but the last a multiple of 32 rows, so no row tile
// straddles two.  Otherwise, one launch each at its offset.
int launch_gemm_q4_0_stacked(mrml_hip_ctx *ctx, const void *const *w, const int32_t *rows, int n, const void *gpack,
                             float *y, int32_t cols, int32_t batch, int32_t ldy, bool relaxed)
{
    if (n < 1 || n > kGemmMaxMats) return fail(ctx, MRML_HIP_E_INVALID, "gemm_q4_0: %d stacked matrices", n);
    int total = 0;
    bool tiles = true;
    for (int m = 0; m < n; ++m) {
        total += rows[m];
        tiles = tiles && (m + 1 == n || rows[m] % 32 == 0);
    }
    if (!tiles) {
        int off = 0;
        for (int m = 0; m < n; ++m) {
            if (int rc = launch_gemm_q4_0(ctx, w[m], gpack, y + off, rows[m], cols, batch, ldy ? ldy : total, relaxed))
                return rc;
            off += rows[m];
        }
        return MRML_HIP_OK;
    }
    GemmMats mats{};
    for (int m = 0; m < n; ++m) {
        mats.w[m] = (const uint8_t *)w[m];
        mats.rows[m] = rows[m];
    }
    mats.n = n;
    return launch_gemm_mats(ctx, mats, gpack, y, total, cols, batch, ldy, relaxed);
}

}  // namespace mrml
