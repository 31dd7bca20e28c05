// device.h -- gfx950 device helpers shared by the kernels.
//
// Every kernel translation unit is compiled with -ffp-contract=off: the
// reference rounds each product and each sum separately (Rust never fuses
// a*b+c), and bit-exact matvec outputs depend on the same two roundings here.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

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
    uint32_t bits = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (bits >> 31) & 1u;
    int32_t exp = (int32_t)((bits >> 23) & 0xffu);
    uint32_t mant = bits & 0x7fffffu;
    if (exp == 255) return (sign << 15) | (mant == 0 ? 0x7c00u : 0x7e00u);
    int32_t e16 = exp - 127 + 15;
    if (e16 >= 31) return (sign << 15) | 0x7c00u;
    if (e16 <= 0) return 0u;
    return (sign << 15) | ((uint32_t)e16 << 10) | (mant >> 13);
}

// f32 -> f16, IEEE round-to-nearest-even (hardware conversion).
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f)
{
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
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

// ops.rs:101-104 evaluated in the same order (contraction is off):
// (0.5*x) * (1 + tanh(k*(x + ((0.044715*x)*x)*x))).
__device__ __forceinline__ float gelu_tanh(float x)
{
    const float k = 0.7978845608f;
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}

}  // namespace mrml
