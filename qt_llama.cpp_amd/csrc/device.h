// device.h -- gfx950 device helpers shared by the kernels.
//
// Every kernel translation unit is compiled with -ffp-contract=off: the
// reference rounds each product and each sum separately (Rust never fuses
// a*b+c), and bit-exact matvec outputs depend on the same two roundings here.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "libm_f32.h"

namespace mrml {

// Backend activation pack for n = 32*nb values (written by the quantiser):
//   int8  q[nb][32]   at byte 0
//   float d[nb]       at byte nb*32   (the f16 block scale, widened exactly)
//   int32 s[nb]       at byte nb*36   (sum of the block's 32 quants)
struct ActPack {
    const int8_t *q;
    const float *d;
    const int32_t *s;
};
__host__ __device__ inline size_t act_pack_bytes(int nb) { return (size_t)nb * 40; }

// f16 bits -> f32.  The hardware conversion is exact for every half,
// subnormals included, as is the reference's bitwise routine (quant.rs:47-77).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h)
{
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;
}

// f32 -> f16 by truncation (quant.rs:81-104): mantissa >> 13, values below
// the f16 normal range -> +0, overflow -> +-Inf, NaN -> sign|0x7e00.
__device__ __forceinline__ uint32_t f32_to_f16_trunc(float f)
{
    // every case formed, then selected (as branches they cost exec-mask
    // switches on the quantisers' critical path)
    const uint32_t bits = __builtin_bit_cast(uint32_t, f);
    const uint32_t sgn = (bits >> 16) & 0x8000u;
    const int32_t exp = (int32_t)((bits >> 23) & 0xffu);
    const uint32_t mant = bits & 0x7fffffu;
    const int32_t e16 = exp - 127 + 15;
    uint32_t special = sgn | (exp == 255 && mant != 0 ? 0x7e00u : 0x7c00u);  // NaN, or Inf / overflow
    uint32_t normal = sgn | ((uint32_t)e16 << 10) | (mant >> 13);
    asm volatile("" : "+v"(special), "+v"(normal));  // formed in every lane: the selects stay selects
    return (exp == 255 || e16 >= 31) ? special : (e16 <= 0 ? 0u : normal);
}

// f32 -> f16, IEEE round-to-nearest-even (hardware conversion).
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f)
{
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

// 16-byte load of a weight-quant stream with the non-temporal hint
// (global_load_dwordx4 ... nt).  A matvec reads each quant byte once per
// pass, so the hint keeps the stream from displacing the activations and
// scale words in L2 and the MALL; on gfx950 it raises a 332 MB streaming
// read from ~6.0 to ~6.7 TB/s.  Scale and header words stay cached loads:
// neighbouring lanes share their lines.
__device__ __forceinline__ uint4 load_stream16(const uint4 *p)
{
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Signed 4x8-bit dot product with int32 accumulate (v_dot4_i32_i8).  The
// nibble and int8 products are exact integers.
__device__ __forceinline__ int32_t sdot4(uint32_t a, uint32_t b, int32_t c)
{
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Value of lane (i-1) mod 16 within each 16-lane DPP row (row_ror:1).
__device__ __forceinline__ float dpp_ror1(float v)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
}

// Ordered fold step across the 16 lanes of a DPP row: lane j receives the
// running sum of lane j-1 and adds its own term.  Applied once per
// "iteration" of 16 consecutive blocks, lane 15 ends up holding
// ((...((s + t_0) + t_1) ...) + t_15), the block-order sequential sum of the
// reference (quant.rs:339-366), with every addition rounded separately.
__device__ __forceinline__ float fold16(float s, float t) { return dpp_ror1(s) + t; }

// Reductions over each 32-lane half of the wave, result in every lane of the
// half.  Within a 16-lane DPP row: quad_perm swaps (xor 1, xor 2) and
// row_ror by 4 and 8; the two rows of a half are then combined through
// v_permlane16_swap (gfx950), all in the VALU.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
// Lane l's value and lane l ^ 16's (the other row of its 32-lane half), in
// either order: v_permlane16_swap on two copies of v exchanges the odd rows
// of the first with the even rows of the second, leaving row 0 of each half
// in one result and row 1 in the other.
__device__ __forceinline__ void row_pair(int v, int &a, int &b)
{
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    a = (int)r[0];
    b = (int)r[1];
}

__device__ __forceinline__ float max32(float m)
{
    auto step = [](float a, float b) { return (b > a) ? b : a; };
    m = step(m, __builtin_bit_cast(float, dpp_mov<0xB1>(__builtin_bit_cast(int, m))));   // quad_perm 1,0,3,2
    m = step(m, __builtin_bit_cast(float, dpp_mov<0x4E>(__builtin_bit_cast(int, m))));   // quad_perm 2,3,0,1
    m = step(m, __builtin_bit_cast(float, dpp_mov<0x124>(__builtin_bit_cast(int, m))));  // row_ror:4
    m = step(m, __builtin_bit_cast(float, dpp_mov<0x128>(__builtin_bit_cast(int, m))));  // row_ror:8
    int a, b;
    row_pair(__builtin_bit_cast(int, m), a, b);
    return step(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

// max32 of values that are all >= +0 (never NaN): their bit patterns order
// as the values do, so an unsigned maximum, which takes its DPP operand
// directly, gives the same bits.
__device__ __forceinline__ float max32_nonneg(float m)
{
    auto step = [](uint32_t a, int b) { return a > (uint32_t)b ? a : (uint32_t)b; };
    uint32_t u = __builtin_bit_cast(uint32_t, m);
    u = step(u, dpp_mov<0xB1>((int)u));
    u = step(u, dpp_mov<0x4E>((int)u));
    u = step(u, dpp_mov<0x124>((int)u));
    u = step(u, dpp_mov<0x128>((int)u));
    int a, b;
    row_pair((int)u, a, b);
    return __builtin_bit_cast(float, step((uint32_t)a, b));
}

__device__ __forceinline__ int sum32(int s)
{
    s += dpp_mov<0xB1>(s);
    s += dpp_mov<0x4E>(s);
    s += dpp_mov<0x124>(s);
    s += dpp_mov<0x128>(s);
    int a, b;
    row_pair(s, a, b);
    return a + b;
}

// One Q8_0 block (quant.rs:193-228) held by 32 consecutive lanes, lane l
// owning value l:
//   amax  = max |x| (starts at 0, NaN never wins -- exact in any order)
//   scale = amax / 127          (IEEE division)
//   d     = f32_to_f16 by truncation;  id = scale != 0 ? 1/scale : 0
//   q     = (int8) clamp(roundf(x*id), -128, 127), NaN -> 0
// Returns q; dbits is the f16 scale, qsum the block's quant sum (both
// uniform across the 32 lanes).  Must be called by all 64 lanes of the wave.
__device__ __forceinline__ int q8_0_block32(float v, uint32_t &dbits, int &qsum)
{
    float m = fabsf(v);
    m = (m > 0.0f) ? m : 0.0f;  // NaN -> 0
    m = max32_nonneg(m);        // max is exact in any order
    const float scale = m / 127.0f;
    dbits = f32_to_f16_trunc(scale);
    const float id = (scale != 0.0f) ? 1.0f / scale : 0.0f;
    float r = roundf(v * id);
    r = (r < -128.0f) ? -128.0f : r;
    r = (r > 127.0f) ? 127.0f : r;
    const int q = (r != r) ? 0 : (int)r;
    qsum = sum32(q);
    return q;
}

// One Q4_0 block (quant.rs:372-389) held by 32 consecutive lanes, lane l
// owning value l:
//   amax    = max |x| (f32::max from 0: NaN never wins -- exact in any order)
//   scale   = amax > 0 ? amax / 8 : 0;  d = f32_to_f16 by truncation
//   inverse = scale > 0 ? 1 / scale : 0
//   q       = clamp(round(x * inverse) as i32, -8, 7) + 8 (round half away
//             from zero; the cast saturates, NaN -> 0)
// Returns q (0..15); dbits is the f16 scale (uniform across the 32 lanes).
// Must be called by all 64 lanes of the wave.
__device__ __forceinline__ int q4_0_block32(float v, uint32_t &dbits)
{
    float m = fabsf(v);
    m = (m > 0.0f) ? m : 0.0f;  // NaN -> 0
    m = max32_nonneg(m);
    const float scale = m > 0.0f ? m / 8.0f : 0.0f;
    dbits = f32_to_f16_trunc(scale);
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    float r = roundf(v * inv);
    r = (r < -8.0f) ? -8.0f : r;  // +-inf saturate to the clamp's ends
    r = (r > 7.0f) ? 7.0f : r;
    return ((r != r) ? 0 : (int)r) + 8;
}

// Reductions over each aligned group of 8 lanes (quad_perm xor 1, xor 2, then
// row_half_mirror, which maps each quad onto the other quad of its 8 lanes;
// after the quad steps every lane of a quad holds the same value).
__device__ __forceinline__ float max8(float m)
{
    auto step = [](float a, float b) { return (b > a) ? b : a; };
    m = step(m, __builtin_bit_cast(float, dpp_mov<0xB1>(__builtin_bit_cast(int, m))));
    m = step(m, __builtin_bit_cast(float, dpp_mov<0x4E>(__builtin_bit_cast(int, m))));
    return step(m, __builtin_bit_cast(float, dpp_mov<0x141>(__builtin_bit_cast(int, m))));
}

__device__ __forceinline__ int sum8(int s)
{
    s += dpp_mov<0xB1>(s);
    s += dpp_mov<0x4E>(s);
    return s + dpp_mov<0x141>(s);
}

__device__ __forceinline__ int q8_0_value(float v, float id)
{
    float r = roundf(v * id);
    r = (r < -128.0f) ? -128.0f : r;
    r = (r > 127.0f) ? 127.0f : r;
    return (r != r) ? 0 : (int)r;
}

// The same Q8_0 block rule with the block held by 8 consecutive lanes, lane l
// owning values 4l..4l+3 (one float4).  Returns the lane's 4 quants packed
// little-endian in a dword; dbits and qsum are uniform across the 8 lanes.
// Must be called by all 64 lanes of the wave.
__device__ __forceinline__ uint32_t q8_0_block8x4(float4 v, uint32_t &dbits, int &qsum)
{
    auto amag = [](float x) {
        const float a = fabsf(x);
        return (a > 0.0f) ? a : 0.0f;  // NaN -> 0
    };
    float m = amag(v.x);
    m = fmaxf(m, amag(v.y));
    m = fmaxf(m, amag(v.z));
    m = fmaxf(m, amag(v.w));
    m = max8(m);
    const float scale = m / 127.0f;
    dbits = f32_to_f16_trunc(scale);
    const float id = (scale != 0.0f) ? 1.0f / scale : 0.0f;
    const int q0 = q8_0_value(v.x, id), q1 = q8_0_value(v.y, id);
    const int q2 = q8_0_value(v.z, id), q3 = q8_0_value(v.w, id);
    qsum = sum8(q0 + q1 + q2 + q3);
    return (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
           ((uint32_t)q3 << 24);
}

// ---- split-nibble activation blocks for the Q4_0 block dot ------------------
// Word i < 4 of a Q4_0 block holds weight q[4i+k] in the low and q[16+4i+k]
// in the high nibble of byte k.  For the Q8_0 quant words x = a[4i..4i+3]
// and y = a[16+4i..16+4i+3] of the activation block:
//   lo_i: nibble 2k = a[4i+k] & 15,  nibble 2k+1 = a[16+4i+k] & 15
//   hi_i: the same nibbles of a >> 4 (4-bit two's complement)
// so every value is a = 16*hi + lo, and with c = -8 * sum(a & 15) over the
// block the exact block dot is
//   sum_k (q_k - 8) * a_k = 16 * sdot8(w ^ 0x88888888, hi) + udot8(w, lo) + c
// (w ^ 0x88888888 holds q - 8 as signed nibbles): 8 dot8 and 4 xor per block
// on the raw weight words, no nibble unpacking.
constexpr uint32_t kLoNib = 0x0F0F0F0Fu;
__device__ __forceinline__ uint32_t split_lo(uint32_t x, uint32_t y) { return (x & kLoNib) | ((y & kLoNib) << 4); }
__device__ __forceinline__ uint32_t split_hi(uint32_t x, uint32_t y) { return ((x >> 4) & kLoNib) | (y & ~kLoNib); }
// sum over the 4 values of a quant word of (a & 15)
__device__ __forceinline__ int lo_nib_sum(uint32_t x)
{
    return (int)__builtin_amdgcn_udot4(x & kLoNib, 0x01010101u, 0u, false);
}

// Lane l of an aligned 8-lane group holds quant word l of one block (q8_0_block8x4
// layout).  Returns split word l of the block (lo_l for l < 4, hi_{l-4}
// above: the word at the same position of the split block) and c in every
// lane of the group.  Must be called by all 64 lanes of the wave.
__device__ __forceinline__ uint32_t q8_split8(uint32_t q, int l, int &c)
{
    const uint32_t p = (uint32_t)__builtin_amdgcn_ds_swizzle((int)q, 0x101F);  // word l ^ 4 (xor mask 4)
    c = -8 * sum8(lo_nib_sum(q));
    return l < 4 ? split_lo(q, p) : split_hi(p, q);
}

// Exact Q4_0 block dot (sum (q-8)*a) of weight words w with a split block.
__device__ __forceinline__ int32_t q4_0_isum_split(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint32_t lo0,
                                                   uint32_t lo1, uint32_t lo2, uint32_t lo3, uint32_t hi0,
                                                   uint32_t hi1, uint32_t hi2, uint32_t hi3, int32_t c)
{
    constexpr uint32_t k8 = 0x88888888u;
    int32_t sh = __builtin_amdgcn_sdot8((int)(w0 ^ k8), (int)hi0, 0, false);
    sh = __builtin_amdgcn_sdot8((int)(w1 ^ k8), (int)hi1, sh, false);
    sh = __builtin_amdgcn_sdot8((int)(w2 ^ k8), (int)hi2, sh, false);
    sh = __builtin_amdgcn_sdot8((int)(w3 ^ k8), (int)hi3, sh, false);
    uint32_t sl = __builtin_amdgcn_udot8(w0, lo0, (uint32_t)c, false);  // wraps: c < 0, the total fits
    sl = __builtin_amdgcn_udot8(w1, lo1, sl, false);
    sl = __builtin_amdgcn_udot8(w2, lo2, sl, false);
    sl = __builtin_amdgcn_udot8(w3, lo3, sl, false);
    return (int32_t)(((uint32_t)sh << 4) + sl);
}

// Stage an activation pack (Q8_0 planes, nb blocks, 16-byte aligned) into
// LDS in split-nibble form (device.h) with one wave, one block per lane;
// every load of a batch is issued before the first block is converted, so
// the copy costs one L2 round trip per 64*kBatch blocks.
// With ISSUE_BARRIER the wave joins one workgroup barrier (s_barrier, no
// memory fence) right after issuing its loads: compute waves that wait on
// that barrier before issuing their weight loads then queue behind the
// pack's loads in the CU's memory pipeline instead of ahead of them (an L2
// hit issued after a CU's worth of HBM misses waits for most of them).  The
// pack is then one batch: nb <= kStageMax, checked by the launchers.
constexpr int kStageBatch = 5, kStageMax = 64 * kStageBatch;

//
// With KQ (the Q4_K matvec, whose quants q = 0..15 carry no -8 offset) the
// block constant is c = 128 * sum(hi) = 8 * sum(a) - 8 * sum(lo), so that
// q4_0_isum_split returns sum q*a, and a fourth plane at nb*40 holds the
// block sums sum(a) (the min term's bsum) as floats, exact (|sum| <= 32*127):
// nb*44 bytes in all.
// nstage >= 0 stages only blocks [0, nstage) (the rest of the LDS pack is
// written by someone else); the layout stays that of nb blocks.
template <bool ISSUE_BARRIER = false, bool KQ = false>
__device__ __forceinline__ void stage_split_pack(const uint8_t *src, uint8_t *lds, int nb, int nstage = -1)
{
    const int lim = nstage >= 0 && nstage < nb ? nstage : nb;
    constexpr int kBatch = kStageBatch;
    const int lane = threadIdx.x & 63;
    const uint4 *sq = reinterpret_cast<const uint4 *>(src);
    const float *sd = reinterpret_cast<const float *>(src + (size_t)nb * 32);
    uint4 *dq = reinterpret_cast<uint4 *>(lds);
    float *dd = reinterpret_cast<float *>(lds + nb * 32);
    int32_t *dc = reinterpret_cast<int32_t *>(lds + nb * 36);
    const int32_t *ss = reinterpret_cast<const int32_t *>(src + (size_t)nb * 36);
    float *dsum = reinterpret_cast<float *>(lds + nb * 40);
    const int nbatch = ISSUE_BARRIER ? 64 * kBatch : nb;  // one pass with the barrier (exactly one s_barrier)
    for (int b0 = 0; b0 < nbatch; b0 += 64 * kBatch) {
        uint4 x[kBatch], y[kBatch];
        float d[kBatch];
        int32_t bs[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            if (b0 + k * 64 >= nb) break;  // wave-uniform: batches past the pack issue no loads
            int b = b0 + k * 64 + lane;
            b = b < nb ? b : nb - 1;
            x[k] = sq[2 * b];
            y[k] = sq[2 * b + 1];
            d[k] = sd[b];
            if constexpr (KQ) bs[k] = ss[b];
        }
        if constexpr (ISSUE_BARRIER) __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int b = b0 + k * 64 + lane;
            if (b < lim) {
                const uint4 lo = make_uint4(split_lo(x[k].x, y[k].x), split_lo(x[k].y, y[k].y),
                                            split_lo(x[k].z, y[k].z), split_lo(x[k].w, y[k].w));
                const uint4 hi = make_uint4(split_hi(x[k].x, y[k].x), split_hi(x[k].y, y[k].y),
                                            split_hi(x[k].z, y[k].z), split_hi(x[k].w, y[k].w));
                dq[2 * b] = lo;
                dq[2 * b + 1] = hi;
                dd[b] = d[k];
                const int c = -8 * (lo_nib_sum(x[k].x) + lo_nib_sum(x[k].y) + lo_nib_sum(x[k].z) + lo_nib_sum(x[k].w) +
                                    lo_nib_sum(y[k].x) + lo_nib_sum(y[k].y) + lo_nib_sum(y[k].z) + lo_nib_sum(y[k].w));
                if constexpr (KQ) {
                    dc[b] = c + 8 * bs[k];
                    dsum[b] = (float)bs[k];
                } else {
                    dc[b] = c;
                }
            }
        }
    }
}

// ops.rs:101-104 evaluated in the same order (contraction is off):
// (0.5*x) * (1 + tanh(k*(x + ((0.044715*x)*x)*x))), with the host C
// library's tanhf reproduced bit for bit (libm_f32.h).
__device__ __forceinline__ float gelu_tanh(float x)
{
    const float k = 0.7978845608f;
    return 0.5f * x * (1.0f + mrml_libm::tanhf(k * (x + 0.044715f * x * x * x)));
}

// GEMM pack of `batch` tokens x nb blocks, groups of 32 tokens (the last
// group zero-padded):
//   int8  q[g][b][h][t][16]  at byte 0              (h = K half, t = token in group)
//   f32   d[g][b][t]         at byte ngroups*nb*1024
__host__ __device__ inline int gemm_groups(int batch) { return (batch + 31) / 32; }

// Writes token m's block b (8 lanes, lane l holding quants 4l..4l+3 packed in
// q) into the GEMM pack.
__device__ __forceinline__ void gemm_pack_put(uint8_t *gp, int ngroups, int nb, int m, int b, int l, uint32_t q,
                                              float d)
{
    const int g = m >> 5, t = m & 31, h = l >> 2;
    const size_t gb = (size_t)g * nb + b;
    reinterpret_cast<uint32_t *>(gp + ((gb * 64 + 32 * h + t) * 16))[l & 3] = q;
    if (l == 0) reinterpret_cast<float *>(gp + (size_t)ngroups * nb * 1024)[gb * 32 + t] = d;
}

}  // namespace mrml
