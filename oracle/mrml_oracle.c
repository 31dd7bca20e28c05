/*
 * mrml_oracle.c -- CPU oracle for the MRML decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP backend is compared against,
 * and the CPU baseline bench.py times beside it.  Never linked into, loaded
 * by, or called from the product library.
 *
 * Plain-C restatement of the reference CPU kernels of
 * mitchellrenouf/QT_llama.cpp (crates/mrml-tensor/src/quant.rs, ops.rs,
 * parallel.rs, kv_cache.rs, model.rs).  Build with -ffp-contract=off and
 * without fast-math: every float operation below rounds once, in the order
 * the Rust source evaluates it (Rust never fuses a*b+c).
 *
 * Parity pins per function (tests/test_oracle.py):
 *   f16 conversions     KATs + numpy float16 (RNE) on exactly-representable
 *                       values + exhaustive round trip of all 65536 halves
 *   Q8_0 quantiser      quant_test.rs:3-22 round trip, all-ones closed form,
 *                       roundf tie cases, brute force vs numpy
 *   Q4_0 x Q8_0 dot     quant_test.rs:24-57, closed forms of
 *                       examples/cuda_prefill_primitives.rs:23-49, ISA
 *                       variants bit-equal (quant.rs:411-432), float64
 *                       dequantised dot, numpy float32 sequential fold
 *   matvec              ops_test.rs:116-140 bit equality of the two entry points
 *   Q8_0 x Q8_0 dot     quant_test.rs:59-76, ops_test.rs:188-237 softcap
 *   rms_norm / rope /   ops_test.rs:79-88, 142-158, closed forms
 *   softmax / gelu
 *   Q4_K                build-defined (GGUF layout): brute force against an
 *                       independent numpy dequantiser, float64 dot
 *   attention, step     build-defined compositions; pinned through their
 *                       parts and closed forms (uniform softmax, pos 0 RoPE)
 */
#include "mrml_oracle.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>
#include <omp.h>

#if defined(__x86_64__)
#include <immintrin.h>
#include <cpuid.h>
#endif

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* ------------------------------------------------------------------------ */
/* quant.rs:47-77 -- exact half -> single, subnormals normalised by a loop.  */
float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    if (exp == 0) {
        if (mant == 0) return bits_f32(sign << 31);
        uint32_t m = mant, e = 0;
        while ((m & 0x400u) == 0) { m <<= 1; e++; }
        m &= 0x3ffu;
        uint32_t exp_f32 = 127u - 15u + 1u - e;
        return bits_f32((sign << 31) | (exp_f32 << 23) | (m << 13));
    }
    if (exp == 31) {
        if (mant == 0) return bits_f32((sign << 31) | (0xffu << 23));
        return bits_f32((sign << 31) | (0xffu << 23) | (mant << 13));
    }
    return bits_f32((sign << 31) | ((exp + (127u - 15u)) << 23) | (mant << 13));
}

/* quant.rs:81-104 -- single -> half by TRUNCATION: mantissa >> 13, no
 * rounding; results below the f16 normal range become +0 (sign dropped);
 * overflow -> +-Inf; NaN -> sign|0x7e00. */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t bits = f32_bits(f);
    uint16_t sign = (uint16_t)((bits >> 31) & 1u);
    int32_t exp = (int32_t)((bits >> 23) & 0xffu);
    uint32_t mant = bits & 0x7fffffu;
    if (exp == 255) return (uint16_t)((sign << 15) | (mant == 0 ? 0x7c00 : 0x7e00));
    int32_t exp16 = exp - 127 + 15;
    if (exp16 >= 31) return (uint16_t)((sign << 15) | 0x7c00);
    if (exp16 <= 0) return 0;
    return (uint16_t)((sign << 15) | ((uint32_t)exp16 << 10) | (mant >> 13));
}

/* IEEE 754 round-to-nearest-even single -> half (build-defined KV store). */
uint16_t orc_f32_to_f16_rne(float f)
{
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to Inf */
    uint32_t e = a >> 23;
    if (e < 113) {                                           /* f16 subnormal or zero */
        if (e < 102) return sign;                            /* < 2^-25 (incl. the tie) */
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                           /* 14..24 */
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (a - (112u << 23)) >> 13;                   /* exponent + mantissa */
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

/* ------------------------------------------------------------------------ */
/* quant.rs:193-228 */
void orc_quantize_q8_0(const float *src, uint8_t *dst, size_t n)
{
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const float *s = src + b * 32;
        uint8_t *d = dst + b * 34;
        float max_val = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(s[i]);
            if (a > max_val) max_val = a;
        }
        float scale = max_val / 127.0f;
        wr16(d, orc_f32_to_f16(scale));
        float id = scale != 0.0f ? 1.0f / scale : 0.0f;
        for (int i = 0; i < 32; i++) {
            float v = roundf(s[i] * id);           /* libm roundf: ties away from 0 */
            if (v < -128.0f) v = -128.0f;          /* f32::clamp(-128, 127) */
            if (v > 127.0f) v = 127.0f;
            int8_t q = isnan(v) ? 0 : (int8_t)v;   /* Rust `as i8`: NaN -> 0 */
            d[2 + i] = (uint8_t)q;
        }
    }
}

/* quant.rs:166-190 */
void orc_dequantize_q8_0(const uint8_t *src, float *dst, size_t n)
{
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *s = src + b * 34;
        float d = orc_f16_to_f32(rd16(s));
        for (int i = 0; i < 32; i++) dst[b * 32 + i] = (float)(int8_t)s[2 + i] * d;
    }
}

/* quant.rs:135-163 */
void orc_dequantize_q4_0(const uint8_t *src, float *dst, size_t n)
{
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *s = src + b * 18;
        float d = orc_f16_to_f32(rd16(s));
        for (int i = 0; i < 16; i++) {
            uint8_t byte = s[2 + i];
            dst[b * 32 + i] = (float)((int)(byte & 0x0f) - 8) * d;
            dst[b * 32 + i + 16] = (float)((int)(byte >> 4) - 8) * d;
        }
    }
}

/* quant.rs:372-389 */
void orc_quantize_q4_0(const float *src, uint8_t *dst, size_t n)
{
    for (size_t b = 0; b < n / 32; b++) {
        const float *v = src + b * 32;
        float max_abs = 0.0f;
        for (int i = 0; i < 32; i++) max_abs = fmaxf(max_abs, fabsf(v[i])); /* f32::max */
        float scale = max_abs > 0.0f ? max_abs / 8.0f : 0.0f;
        uint8_t *d = dst + b * 18;
        wr16(d, orc_f32_to_f16(scale));
        float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int i = 0; i < 16; i++) {
            float rl = roundf(v[i] * inverse), rh = roundf(v[i + 16] * inverse);
            /* `as i32` saturates and maps NaN to 0; then clamp(-8, 7) */
            int32_t lo = isnan(rl) ? 0 : (rl >= 2147483647.0f ? 2147483647 : (rl <= -2147483648.0f ? (-2147483647 - 1) : (int32_t)rl));
            int32_t hi = isnan(rh) ? 0 : (rh >= 2147483647.0f ? 2147483647 : (rh <= -2147483648.0f ? (-2147483647 - 1) : (int32_t)rh));
            lo = lo < -8 ? -8 : (lo > 7 ? 7 : lo);
            hi = hi < -8 ? -8 : (hi > 7 ? 7 : hi);
            d[2 + i] = (uint8_t)((uint8_t)(lo + 8) | (uint8_t)((hi + 8) << 4));
        }
    }
}

/* ------------------------------------------------------------------------ */
/* CPU feature detection, quant.rs:11-43 and 394-404. */
#if defined(__x86_64__)
static int x86_avx_state_enabled(void)
{
    unsigned a, b, c, d;
    if (!__get_cpuid(1, &a, &b, &c, &d)) return 0;
    if (!((c & (1u << 28)) && (c & (1u << 27)))) return 0;
    unsigned lo, hi;
    __asm__ volatile("xgetbv" : "=a"(lo), "=d"(hi) : "c"(0));
    return (lo & 6u) == 6u;
}
static int have_avx2(void)
{
    unsigned a, b, c, d;
    if (!x86_avx_state_enabled()) return 0;
    __cpuid_count(7, 0, a, b, c, d);
    return (b & (1u << 5)) != 0;
}
static int have_avx_vnni(void)
{
    unsigned a, b, c, d;
    if (!x86_avx_state_enabled()) return 0;
    __cpuid_count(7, 1, a, b, c, d);
    return (a & (1u << 4)) != 0;
}
#else
static int have_avx2(void) { return 0; }
static int have_avx_vnni(void) { return 0; }
#endif

int orc_host_isa(void)
{
    if (have_avx_vnni()) return 2;
    if (have_avx2()) return 1;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* quant.rs:335-369 -- scalar Q4_0 x Q8_0.  sum += (float)isum * (dw*da). */
static float dot_q4_0_q8_0_scalar(const uint8_t *w, const uint8_t *a, size_t n)
{
    float sum = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *wb = w + b * 18, *ab = a + b * 34;
        float d_w = orc_f16_to_f32(rd16(wb)), d_a = orc_f16_to_f32(rd16(ab));
        int32_t block_sum = 0;
        for (int i = 0; i < 16; i++) {
            uint8_t byte = wb[2 + i];
            int32_t q0 = (int32_t)(byte & 0x0f) - 8, q1 = (int32_t)(byte >> 4) - 8;
            int32_t a0 = (int8_t)ab[2 + i], a1 = (int8_t)ab[2 + i + 16];
            block_sum += q0 * a0 + q1 * a1;
        }
        sum += (float)block_sum * (d_w * d_a);
    }
    return sum;
}

#if defined(__x86_64__)
/* quant.rs:272-332 -- AVX2.  The integer block sum is exact, and the float
 * update is the scalar one, so the result is bit-identical to scalar. */
__attribute__((target("avx2")))
static float dot_q4_0_q8_0_avx2(const uint8_t *w, const uint8_t *a, size_t n)
{
    float sum = 0.0f;
    const __m128i mask_low = _mm_set1_epi8(0x0f), eight = _mm_set1_epi8(8);
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *wb = w + b * 18, *ab = a + b * 34;
        float d_w = orc_f16_to_f32(rd16(wb)), d_a = orc_f16_to_f32(rd16(ab));
        __m128i q4 = _mm_loadu_si128((const __m128i *)(wb + 2));
        __m128i q8l = _mm_loadu_si128((const __m128i *)(ab + 2));
        __m128i q8h = _mm_loadu_si128((const __m128i *)(ab + 18));
        __m128i lo = _mm_sub_epi8(_mm_and_si128(q4, mask_low), eight);
        __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(q4, 4), mask_low), eight);
        __m128i p0 = _mm_madd_epi16(_mm_cvtepi8_epi16(lo), _mm_cvtepi8_epi16(q8l));
        __m128i p1 = _mm_madd_epi16(_mm_cvtepi8_epi16(_mm_srli_si128(lo, 8)), _mm_cvtepi8_epi16(_mm_srli_si128(q8l, 8)));
        __m128i p2 = _mm_madd_epi16(_mm_cvtepi8_epi16(hi), _mm_cvtepi8_epi16(q8h));
        __m128i p3 = _mm_madd_epi16(_mm_cvtepi8_epi16(_mm_srli_si128(hi, 8)), _mm_cvtepi8_epi16(_mm_srli_si128(q8h, 8)));
        __m128i s = _mm_add_epi32(_mm_add_epi32(p0, p1), _mm_add_epi32(p2, p3));
        int32_t acc[4];
        _mm_storeu_si128((__m128i *)acc, s);
        int32_t block_sum = acc[0] + acc[1] + acc[2] + acc[3];
        sum += (float)block_sum * (d_w * d_a);
    }
    return sum;
}

/* quant.rs:443-479 -- AVX-VNNI (vpdpwssd on sign-extended 16-bit lanes). */
__attribute__((target("avx2,avxvnni")))
static float dot_q4_0_q8_0_vnni(const uint8_t *w, const uint8_t *a, size_t n)
{
    float sum = 0.0f;
    const __m128i mask = _mm_set1_epi8(0x0f), eight = _mm_set1_epi8(8);
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *wb = w + b * 18, *ab = a + b * 34;
        float scale = orc_f16_to_f32(rd16(wb)) * orc_f16_to_f32(rd16(ab));
        __m128i packed = _mm_loadu_si128((const __m128i *)(wb + 2));
        __m128i lo = _mm_sub_epi8(_mm_and_si128(packed, mask), eight);
        __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(packed, 4), mask), eight);
        __m128i q8l = _mm_loadu_si128((const __m128i *)(ab + 2));
        __m128i q8h = _mm_loadu_si128((const __m128i *)(ab + 18));
        __m256i dot = _mm256_dpwssd_avx_epi32(_mm256_setzero_si256(), _mm256_cvtepi8_epi16(lo), _mm256_cvtepi8_epi16(q8l));
        dot = _mm256_dpwssd_avx_epi32(dot, _mm256_cvtepi8_epi16(hi), _mm256_cvtepi8_epi16(q8h));
        int32_t lanes[8];
        _mm256_storeu_si256((__m256i *)lanes, dot);
        int32_t isum = 0;
        for (int i = 0; i < 8; i++) isum += lanes[i];
        sum += (float)isum * scale;
    }
    return sum;
}
#endif

float orc_vec_dot_q4_0_q8_0(const uint8_t *w, const uint8_t *a, size_t n, int isa)
{
    if (isa < 0) isa = orc_host_isa();
#if defined(__x86_64__)
    if (isa == 2) return have_avx_vnni() ? dot_q4_0_q8_0_vnni(w, a, n) : NAN;
    if (isa == 1) return have_avx2() ? dot_q4_0_q8_0_avx2(w, a, n) : NAN;
#else
    if (isa != 0) return NAN;
#endif
    return dot_q4_0_q8_0_scalar(w, a, n);
}

void orc_block_isums_q4_0_q8_0(const uint8_t *w, const uint8_t *a, size_t n, int32_t *isum)
{
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *wb = w + b * 18, *ab = a + b * 34;
        int32_t s = 0;
        for (int i = 0; i < 16; i++) {
            s += ((int32_t)(wb[2 + i] & 0x0f) - 8) * (int8_t)ab[2 + i];
            s += ((int32_t)(wb[2 + i] >> 4) - 8) * (int8_t)ab[18 + i];
        }
        isum[b] = s;
    }
}

void orc_block_isums_q8_0_q8_0(const uint8_t *x, const uint8_t *y, size_t n, int32_t *isum)
{
    for (size_t b = 0; b < n / 32; b++) {
        int32_t s = 0;
        for (int i = 0; i < 32; i++) s += (int8_t)x[b * 34 + 2 + i] * (int8_t)y[b * 34 + 2 + i];
        isum[b] = s;
    }
}

/* quant.rs:563-577 */
static float dot_q8_0_q8_0_scalar(const uint8_t *x, const uint8_t *y, size_t n)
{
    float sum = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        size_t off = b * 34;
        float dx = orc_f16_to_f32(rd16(x + off)), dy = orc_f16_to_f32(rd16(y + off));
        int32_t block_sum = 0;
        for (int i = 0; i < 32; i++) block_sum += (int8_t)x[off + 2 + i] * (int8_t)y[off + 2 + i];
        sum += (float)block_sum * (dx * dy);
    }
    return sum;
}

#if defined(__x86_64__)
/* quant.rs:497-530 -- same fold as scalar. */
__attribute__((target("avx2,avxvnni")))
static float dot_q8_0_q8_0_vnni(const uint8_t *x, const uint8_t *y, size_t n)
{
    float sum = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        size_t off = b * 34;
        float scale = orc_f16_to_f32(rd16(x + off)) * orc_f16_to_f32(rd16(y + off));
        __m128i xl = _mm_loadu_si128((const __m128i *)(x + off + 2));
        __m128i xh = _mm_loadu_si128((const __m128i *)(x + off + 18));
        __m128i yl = _mm_loadu_si128((const __m128i *)(y + off + 2));
        __m128i yh = _mm_loadu_si128((const __m128i *)(y + off + 18));
        __m256i dot = _mm256_dpwssd_avx_epi32(_mm256_setzero_si256(), _mm256_cvtepi8_epi16(xl), _mm256_cvtepi8_epi16(yl));
        dot = _mm256_dpwssd_avx_epi32(dot, _mm256_cvtepi8_epi16(xh), _mm256_cvtepi8_epi16(yh));
        int32_t lanes[8];
        _mm256_storeu_si256((__m256i *)lanes, dot);
        int32_t isum = 0;
        for (int i = 0; i < 8; i++) isum += lanes[i];
        sum += (float)isum * scale;
    }
    return sum;
}

/* quant.rs:532-561 -- AVX2-only hosts: eight f32 lane accumulators, lane j
 * holding the madd partials of elements {2j,2j+1,16+2j,17+2j}; the lanes are
 * summed at the end with Iterator::sum (a fold from -0.0). */
__attribute__((target("avx2")))
static float dot_q8_0_q8_0_avx2(const uint8_t *x, const uint8_t *y, size_t n)
{
    __m256 accum = _mm256_setzero_ps();
    for (size_t b = 0; b < n / 32; b++) {
        size_t off = b * 34;
        float dx = orc_f16_to_f32(rd16(x + off)), dy = orc_f16_to_f32(rd16(y + off));
        __m256i xv = _mm256_loadu_si256((const __m256i *)(x + off + 2));
        __m256i yv = _mm256_loadu_si256((const __m256i *)(y + off + 2));
        __m256i x_lo = _mm256_cvtepi8_epi16(_mm256_castsi256_si128(xv));
        __m256i x_hi = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(xv, 1));
        __m256i y_lo = _mm256_cvtepi8_epi16(_mm256_castsi256_si128(yv));
        __m256i y_hi = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(yv, 1));
        __m256i products = _mm256_add_epi32(_mm256_madd_epi16(x_lo, y_lo), _mm256_madd_epi16(x_hi, y_hi));
        __m256 scaled = _mm256_mul_ps(_mm256_cvtepi32_ps(products), _mm256_set1_ps(dx * dy));
        accum = _mm256_add_ps(accum, scaled);
    }
    float lanes[8];
    _mm256_storeu_ps(lanes, accum);
    float s = -0.0f;
    for (int i = 0; i < 8; i++) s += lanes[i];
    return s;
}
#endif

float orc_vec_dot_q8_0_q8_0(const uint8_t *x, const uint8_t *y, size_t n, int isa)
{
    if (isa < 0) isa = orc_host_isa();
#if defined(__x86_64__)
    if (isa == 2) return have_avx_vnni() ? dot_q8_0_q8_0_vnni(x, y, n) : NAN;
    if (isa == 1) return have_avx2() ? dot_q8_0_q8_0_avx2(x, y, n) : NAN;
#else
    if (isa != 0) return NAN;
#endif
    return dot_q8_0_q8_0_scalar(x, y, n);
}

/* ------------------------------------------------------------------------ */
/* parallel.rs:73-116: jobs = min(workers, ceil(len/min_chunk)), contiguous
 * ranges of ceil(len/jobs) rows; len <= min_chunk runs on the caller. */
#define ROW_LOOP(len, min_chunk, threads, BODY)                                   \
    do {                                                                          \
        size_t len_ = (len);                                                      \
        int workers_ = (threads);                                                 \
        if (workers_ <= 1 || len_ <= (size_t)(min_chunk)) {                       \
            for (size_t r = 0; r < len_; r++) { BODY; }                           \
        } else {                                                                  \
            size_t jobs_ = (len_ + (min_chunk) - 1) / (min_chunk);                \
            if (jobs_ > (size_t)workers_) jobs_ = (size_t)workers_;              \
            size_t chunk_ = (len_ + jobs_ - 1) / jobs_;                           \
            _Pragma("omp parallel num_threads(jobs_)")                            \
            {                                                                     \
                size_t t_ = (size_t)omp_get_thread_num();                         \
                size_t s_ = t_ * chunk_, e_ = s_ + chunk_;                        \
                if (e_ > len_) e_ = len_;                                         \
                for (size_t r = s_; r < e_; r++) { BODY; }                        \
            }                                                                     \
        }                                                                         \
    } while (0)

/* ops.rs:221-260 */
void orc_mat_vec_mul_q4_0_q8_0(const uint8_t *w, const uint8_t *x_q8, float *y,
                               size_t rows, size_t cols, int isa, int threads)
{
    size_t row_bytes = (cols + 31) / 32 * 18;
    if (isa < 0) isa = orc_host_isa();
    ROW_LOOP(rows, 64, threads, y[r] = orc_vec_dot_q4_0_q8_0(w + r * row_bytes, x_q8, cols, isa));
}

/* ops.rs:162-180 */
void orc_mat_vec_mul_q4_0(const uint8_t *w, const float *x, float *y,
                          size_t rows, size_t cols, int isa, int threads)
{
    uint8_t *xq = (uint8_t *)calloc((cols + 31) / 32 * 34, 1);
    orc_quantize_q8_0(x, xq, cols);
    orc_mat_vec_mul_q4_0_q8_0(w, xq, y, rows, cols, isa, threads);
    free(xq);
}

/* model.rs:2842-2861 (vocabulary map, minimum chunk 1024) */
void orc_mat_vec_mul_q8_0_q8_0(const uint8_t *w, const uint8_t *x_q8, float *y,
                               size_t rows, size_t cols, int softcap, int isa, int threads)
{
    size_t row_bytes = (cols + 31) / 32 * 34;
    if (isa < 0) isa = orc_host_isa();
    ROW_LOOP(rows, 1024, threads, {
        float v = orc_vec_dot_q8_0_q8_0(w + r * row_bytes, x_q8, cols, isa);
        y[r] = softcap ? 30.0f * tanhf(v / 30.0f) : v;
    });
}

/* ------------------------------------------------------------------------ */
/* Q4_K, GGUF layout: {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}. */
void orc_q4_k_scale_min(const uint8_t *q, int j, uint8_t *sc, uint8_t *m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void orc_dequantize_q4_k(const uint8_t *src, float *dst, size_t n)
{
    for (size_t sb = 0; sb < n / 256; sb++) {
        const uint8_t *blk = src + sb * 144;
        float d = orc_f16_to_f32(rd16(blk)), dmin = orc_f16_to_f32(rd16(blk + 2));
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        float *out = dst + sb * 256;
        for (int c = 0; c < 4; c++) {
            uint8_t sc, m;
            orc_q4_k_scale_min(scales, 2 * c, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            orc_q4_k_scale_min(scales, 2 * c + 1, &sc, &m);
            float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; l++) {
                out[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0x0f) - m1;
                out[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - m2;
            }
        }
    }
}

float orc_vec_dot_q4_k_q8_0(const uint8_t *w, const uint8_t *a, size_t n)
{
    float sum = 0.0f;
    for (size_t sb = 0; sb < n / 256; sb++) {
        const uint8_t *blk = w + sb * 144;
        float d = orc_f16_to_f32(rd16(blk)), dmin = orc_f16_to_f32(rd16(blk + 2));
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        for (int j = 0; j < 8; j++) {
            const uint8_t *ab = a + (sb * 8 + (size_t)j) * 34;
            float d_a = orc_f16_to_f32(rd16(ab));
            uint8_t sc, m;
            orc_q4_k_scale_min(scales, j, &sc, &m);
            int32_t isum = 0, bsum = 0;
            const uint8_t *q = qs + 32 * (j / 2);
            int shift = (j & 1) ? 4 : 0;
            for (int l = 0; l < 32; l++) {
                int32_t av = (int8_t)ab[2 + l];
                isum += (int32_t)((q[l] >> shift) & 0x0f) * av;
                bsum += av;
            }
            float ds = (d * (float)sc) * d_a;
            float dm = (dmin * (float)m) * d_a;
            float t = (float)isum * ds - (float)bsum * dm;
            sum = sum + t;
        }
    }
    return sum;
}

void orc_mat_vec_mul_q4_k_q8_0(const uint8_t *w, const uint8_t *x_q8, float *y,
                               size_t rows, size_t cols, int threads)
{
    size_t row_bytes = cols / 256 * 144;
    ROW_LOOP(rows, 64, threads, y[r] = orc_vec_dot_q4_k_q8_0(w + r * row_bytes, x_q8, cols));
}

/* ------------------------------------------------------------------------ */
int64_t orc_argmax_f32(const float *x, size_t n)
{
    if (n == 0) return -1;
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (x[i] > x[best] || (isnan(x[best]) && !isnan(x[i]))) best = i;
    return (int64_t)best;
}

/* model.rs:2842-2907 (CPU path of step_generation) */
typedef struct { float s; int32_t id; } orc_cand;

static int orc_cand_before(const orc_cand *a, const orc_cand *b)
{
    return a->s > b->s || (a->s == b->s && a->id < b->id);
}

int32_t orc_vocab_select(const float *logits, size_t vocab, const uint8_t *valid, const int32_t *recent,
                         size_t n_recent, size_t generated_count, int scoring, float temperature, uint64_t pos,
                         size_t k, float *out_scores, int32_t *out_ids, size_t *n_out)
{
    /* the k best candidates, kept sorted (insertion: k is small) */
    orc_cand *best = malloc((k ? k : 1) * sizeof *best);
    size_t nb = 0;
    for (size_t id = 0; id < vocab; id++) {
        if (valid && !valid[id]) continue;
        if (generated_count < 4 && (id == 1 || id == 2 || id == 105 || id == 106)) continue;
        float s = logits[id];
        if (scoring == 0) { /* CPU path: softcap, 3.5 once (model.rs:2852-2856) */
            s = 30.0f * tanhf(s / 30.0f);
            for (size_t r = 0; r < n_recent; r++)
                if (recent[r] == (int32_t)id) { s -= 3.5f; break; }
        } else { /* device path: 1.8 per occurrence (kernels.rs:1114-1121) */
            for (size_t r = 0; r < n_recent; r++)
                if (recent[r] == (int32_t)id) s -= 1.8f;
        }
        if (isnan(s)) continue;
        orc_cand c = {s, (int32_t)id};
        if (nb == k && (k == 0 || !orc_cand_before(&c, &best[k - 1]))) continue;
        size_t at = nb < k ? nb++ : k - 1;
        while (at > 0 && orc_cand_before(&c, &best[at - 1])) { best[at] = best[at - 1]; at--; }
        best[at] = c;
    }
    for (size_t i = 0; i < nb; i++) {
        if (out_scores) out_scores[i] = best[i].s;
        if (out_ids) out_ids[i] = best[i].id;
    }
    if (n_out) *n_out = nb;
    int32_t token = nb ? best[0].id : 506;
    if (nb && temperature > 0.0f) {
        const float max_logit = best[0].s;
        const float temp = temperature > 0.1f ? temperature : 0.1f;
        float *probs = malloc(nb * sizeof *probs);
        float sum_exp = 0.0f;
        for (size_t i = 0; i < nb; i++) {
            probs[i] = expf((best[i].s - max_logit) / temp);
            sum_exp += probs[i];
        }
        if (sum_exp > 0.0f) {
            const float rng = (float)((pos * 6364136223846793005ull + 1ull) >> 33) / (float)UINT32_MAX;
            float acc = 0.0f;
            for (size_t i = 0; i < nb; i++) {
                acc += probs[i] / sum_exp;
                if (rng <= acc) { token = best[i].id; break; }
            }
        }
        free(probs);
    }
    free(best);
    return token;
}

/* ops.rs:24-49 */
void orc_rms_norm(const float *x, const float *w, float eps, float *out, size_t dim)
{
    float sum_sq = 0.0f;
    for (size_t i = 0; i < dim; i++) sum_sq += x[i] * x[i];
    float mean_sq = sum_sq / (float)dim;
    float scale = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < dim; i++) out[i] = w ? x[i] * scale * w[i] : x[i] * scale;
}

/* ops.rs:82-97 */
void orc_rope_1d(float *v, size_t pos, size_t head_dim, float base, float fscale)
{
    size_t half = head_dim / 2;
    for (size_t i = 0; i < half; i++) {
        float theta = (float)pos * fscale / powf(base, (float)(2 * i) / (float)head_dim);
        float c = cosf(theta), s = sinf(theta);
        float v0 = v[i], v1 = v[i + half];
        v[i] = v0 * c - v1 * s;
        v[i + half] = v0 * s + v1 * c;
    }
}

/* ops.rs:185-208 */
void orc_rope_1d_batched(float *v, size_t pos, size_t n_heads, size_t head_dim,
                         float base, float fscale)
{
    size_t half = head_dim / 2;
    for (size_t i = 0; i < half; i++) {
        float theta = (float)pos * fscale / powf(base, (float)(2 * i) / (float)head_dim);
        float c = cosf(theta), s = sinf(theta);
        for (size_t h = 0; h < n_heads; h++) {
            float *hd = v + h * head_dim;
            float v0 = hd[i], v1 = hd[i + half];
            hd[i] = v0 * c - v1 * s;
            hd[i + half] = v0 * s + v1 * c;
        }
    }
}

/* ops.rs:101-104 */
float orc_gelu_approx(float x)
{
    const float k = 0.7978845608f;
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}

/* ops.rs:107-114 */
void orc_geglu(const float *gate, const float *up, float *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_gelu_approx(gate[i]) * up[i];
}

/* ops.rs:118-120 */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* ops.rs:123-130 */
void orc_swiglu(const float *gate, const float *up, float *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_silu(gate[i]) * up[i];
}

/* ops.rs:133-158 */
void orc_softmax(float *x, size_t n)
{
    if (n == 0) return;
    float max_val = x[0];
    for (size_t i = 1; i < n; i++) if (x[i] > max_val) max_val = x[i];
    float sum_exp = 0.0f;
    for (size_t i = 0; i < n; i++) { float e = expf(x[i] - max_val); x[i] = e; sum_exp += e; }
    if (sum_exp > 0.0f) {
        float inv = 1.0f / sum_exp;
        for (size_t i = 0; i < n; i++) x[i] *= inv;
    }
}

/* ------------------------------------------------------------------------ */
/* model.rs:1457-1590 with the F32-row semantics of kv_cache.rs:72-124
 * (dot: Iterator::sum of a*b from -0.0; accumulate: *dst += p * src) over an
 * f16 cache, times a score scale. */
void orc_attention_f16(const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                       float *out, size_t n_past, size_t n_heads, size_t n_kv_heads,
                       size_t head_dim, float scale)
{
    size_t count = n_past + 1, group = n_heads / n_kv_heads;
    float *scores = (float *)malloc(count * sizeof(float));
    for (size_t h = 0; h < n_heads; h++) {
        size_t kv_h = h / group;
        const float *qh = q + h * head_dim;
        for (size_t t = 0; t < count; t++) {
            const uint16_t *kr = k_cache + (t * n_kv_heads + kv_h) * head_dim;
            float dot = -0.0f;
            for (size_t d = 0; d < head_dim; d++) dot += qh[d] * orc_f16_to_f32(kr[d]);
            scores[t] = dot * scale;
        }
        orc_softmax(scores, count);
        float *oh = out + h * head_dim;
        for (size_t d = 0; d < head_dim; d++) oh[d] = 0.0f;
        for (size_t t = 0; t < count; t++) {
            const uint16_t *vr = v_cache + (t * n_kv_heads + kv_h) * head_dim;
            float p = scores[t];
            for (size_t d = 0; d < head_dim; d++) oh[d] += p * orc_f16_to_f32(vr[d]);
        }
    }
    free(scores);
}

/* ------------------------------------------------------------------------ */
/* KV cache rows in the three formats of KvCacheFormat::cuda_code
 * (kv_cache.rs:16-31): 0 f16 (the build's cache of the F32 format, RNE as
 * the reference GPU stores it), 1 Q8_0, 2 Q4_0.  Bytes of n values. */
size_t orc_kv_row_bytes(size_t n, int fmt)
{
    return fmt == 1 ? n / 32 * 34 : (fmt == 2 ? n / 32 * 18 : n * 2);
}

/* KvCacheRow::from_f32 (kv_cache.rs:54-71): the f16 cache rounds each value
 * to nearest even; Q8_0 and Q4_0 rows are quantize_f32_to_q8_0 /
 * quantize_f32_to_q4_0 of the whole row (blocks of 32 along it). */
void orc_kv_store(const float *x, uint8_t *dst, size_t n, int fmt)
{
    if (fmt == 1) {
        orc_quantize_q8_0(x, dst, n);
    } else if (fmt == 2) {
        orc_quantize_q4_0(x, dst, n);
    } else {
        for (size_t i = 0; i < n; i++) wr16(dst + 2 * i, orc_f32_to_f16_rne(x[i]));
    }
}

/* KvCacheRow::dot_head (kv_cache.rs:73-95) of one head's cached keys:
 *   fmt 0: -0.0 + q[0]*k[0] + ... in d order (the f16 cache widened exactly);
 *   fmt 1 / 2: vec_dot_q8_0_q8_0 / vec_dot_q4_0_q8_0 of the head's K blocks
 *     with q8 = quantize_f32_to_q8_0(q) (model.rs:1530-1531), the scalar fold
 *     (the AVX-VNNI path gives the same bits; quant.rs:406-439). */
float orc_kv_dot_head(const uint8_t *row, const float *q, const uint8_t *q8, size_t head_dim, int fmt)
{
    if (fmt == 1) return dot_q8_0_q8_0_scalar(row, q8, head_dim);
    if (fmt == 2) return dot_q4_0_q8_0_scalar(row, q8, head_dim);
    float dot = -0.0f;
    for (size_t d = 0; d < head_dim; d++) dot += q[d] * orc_f16_to_f32(rd16(row + 2 * d));
    return dot;
}

/* KvCacheRow::add_head_scaled (kv_cache.rs:97-125):
 *   fmt 0: out[d] += p * v[d];
 *   fmt 1: per block b, dd = f16(d_b) * p, out[32b+i] += dd * q_i;
 *   fmt 2: per block b, dd = f16(d_b) * p, out[32b+i] += dd * (lo_i - 8) and
 *          out[32b+16+i] += dd * (hi_i - 8) for byte i. */
void orc_kv_add_head_scaled(const uint8_t *row, float *out, size_t head_dim, float p, int fmt)
{
    if (fmt == 0) {
        for (size_t d = 0; d < head_dim; d++) out[d] += p * orc_f16_to_f32(rd16(row + 2 * d));
        return;
    }
    const size_t bb = fmt == 1 ? 34 : 18;
    for (size_t b = 0; b < head_dim / 32; b++) {
        const uint8_t *blk = row + b * bb;
        const float dd = orc_f16_to_f32(rd16(blk)) * p;
        float *o = out + 32 * b;
        if (fmt == 1) {
            for (int i = 0; i < 32; i++) o[i] += dd * (float)(int8_t)blk[2 + i];
        } else {
            for (int i = 0; i < 16; i++) {
                o[i] += dd * (float)((int)(blk[2 + i] & 15) - 8);
                o[i + 16] += dd * (float)((int)(blk[2 + i] >> 4) - 8);
            }
        }
    }
}

/* Attention over caches in those formats, the CPU loop of model.rs:1526-1547:
 * per query head h (kv head h / (n_heads / n_kv_heads)), score_t =
 * dot_head(k_t) * scale (the reference model's scale is 1.0, which leaves
 * the dot as it is), softmax (ops.rs:133-158), then out = 0 and
 * add_head_scaled(v_t, p_t) position by position.  Caches are
 * [pos][n_kv_heads][head_dim] in the formats' bytes; positions 0..n_past are
 * attended.  With both formats 0 this is orc_attention_f16. */
void orc_attention_kv(const float *q, const uint8_t *k_cache, const uint8_t *v_cache, float *out, size_t n_past,
                      size_t n_heads, size_t n_kv_heads, size_t head_dim, float scale, int k_fmt, int v_fmt)
{
    const size_t count = n_past + 1, group = n_heads / n_kv_heads;
    const size_t k_head = orc_kv_row_bytes(head_dim, k_fmt), v_head = orc_kv_row_bytes(head_dim, v_fmt);
    const size_t k_row = k_head * n_kv_heads, v_row = v_head * n_kv_heads;
    float *scores = (float *)malloc(count * sizeof(float));
    uint8_t *q8 = (uint8_t *)malloc(head_dim / 32 * 34 + 34);
    for (size_t h = 0; h < n_heads; h++) {
        const size_t kv_h = h / group;
        const float *qh = q + h * head_dim;
        if (k_fmt != 0) orc_quantize_q8_0(qh, q8, head_dim);
        for (size_t t = 0; t < count; t++)
            scores[t] = orc_kv_dot_head(k_cache + t * k_row + kv_h * k_head, qh, q8, head_dim, k_fmt) * scale;
        orc_softmax(scores, count);
        float *oh = out + h * head_dim;
        for (size_t d = 0; d < head_dim; d++) oh[d] = 0.0f;
        for (size_t t = 0; t < count; t++)
            orc_kv_add_head_scaled(v_cache + t * v_row + kv_h * v_head, oh, head_dim, scores[t], v_fmt);
    }
    free(q8);
    free(scores);
}

/* ------------------------------------------------------------------------ */
/* Build-defined Gemma-2-2B-shape decode step (composition of the reference
 * ops in the order of model.rs:1185-2260, with Gemma-2's dense GeGLU FFN,
 * sandwich norms, 1/sqrt(head_dim) attention scale and a tied table). */
int64_t orc_gemma2_step(const orc_gemma2 *m, int64_t token, int64_t pos,
                        uint16_t *k_cache, uint16_t *v_cache, float *logits, int threads)
{
    const size_t dim = (size_t)m->dim, hd = (size_t)m->head_dim;
    const size_t qd = (size_t)m->n_heads * hd, kvd = (size_t)m->n_kv_heads * hd;
    const size_t ffn = (size_t)m->ffn_dim, vocab = (size_t)m->vocab;
    const int isa = orc_host_isa();
    float *h = malloc(dim * 4), *xn = malloc(dim * 4), *tmp = malloc(dim * 4);
    float *q = malloc(qd * 4), *k = malloc(kvd * 4), *v = malloc(kvd * 4), *att = malloc(qd * 4);
    float *g = malloc(ffn * 4), *u = malloc(ffn * 4), *act = malloc(ffn * 4);
    size_t maxk = ffn > dim ? ffn : dim;
    if (qd > maxk) maxk = qd;
    uint8_t *xq = malloc(maxk / 32 * 34);
    float *lg = logits ? logits : malloc(vocab * 4);

    /* embedding: dequantised tied row x sqrt(dim) (model.rs:1164-1174,1201,1255-1259) */
    size_t tok = (size_t)(token < 0 ? 0 : (token >= (int64_t)vocab ? (int64_t)vocab - 1 : token));
    if (m->tie_q8) orc_dequantize_q8_0(m->tok_embd + tok * (dim / 32 * 34), h, dim);
    else orc_dequantize_q4_0(m->tok_embd + tok * (dim / 32 * 18), h, dim);
    float es = sqrtf((float)dim);
    for (size_t i = 0; i < dim; i++) h[i] *= es;

    for (int l = 0; l < m->n_layers; l++) {
        orc_rms_norm(h, m->attn_norm[l], m->eps, xn, dim);
        orc_quantize_q8_0(xn, xq, dim);
        orc_mat_vec_mul_q4_0_q8_0(m->wq[l], xq, q, qd, dim, isa, threads);
        orc_mat_vec_mul_q4_0_q8_0(m->wk[l], xq, k, kvd, dim, isa, threads);
        orc_mat_vec_mul_q4_0_q8_0(m->wv[l], xq, v, kvd, dim, isa, threads);
        orc_rope_1d_batched(q, (size_t)pos, (size_t)m->n_heads, hd, m->rope_base, 1.0f);
        orc_rope_1d_batched(k, (size_t)pos, (size_t)m->n_kv_heads, hd, m->rope_base, 1.0f);
        uint16_t *kc = k_cache + (size_t)l * (size_t)m->ctx * kvd;
        uint16_t *vc = v_cache + (size_t)l * (size_t)m->ctx * kvd;
        /* the cache is a ring of ctx rows: position pos lands in row pos % ctx
         * (kernels.rs:1307-1313) and attention reads the last min(pos+1, ctx)
         * positions, oldest first (a sliding window of ctx, kernels.rs:1398-1404) */
        const size_t ctx = (size_t)m->ctx, crow = (size_t)pos % ctx;
        for (size_t i = 0; i < kvd; i++) {
            kc[crow * kvd + i] = orc_f32_to_f16_rne(k[i]);
            vc[crow * kvd + i] = orc_f32_to_f16_rne(v[i]);
        }
        /* windowed layers (model.rs:590, 1465-1467): the last sliding_window
         * positions, unless the layer is a period's last (global) one */
        size_t limit = ctx;
        if (m->sliding_window > 0 && m->swa_period > 0 && l % m->swa_period != m->swa_period - 1 &&
            (size_t)m->sliding_window < ctx)
            limit = (size_t)m->sliding_window;
        const size_t count = (size_t)pos + 1, win = count > limit ? limit : count, start = count - win;
        if (start == 0) {
            orc_attention_f16(q, kc, vc, att, (size_t)pos, (size_t)m->n_heads, (size_t)m->n_kv_heads,
                              hd, m->attn_scale);
        } else {
            uint16_t *wk = malloc(win * kvd * 2), *wv = malloc(win * kvd * 2);
            for (size_t t = 0; t < win; t++) {
                const size_t row = (start + t) % ctx;
                memcpy(wk + t * kvd, kc + row * kvd, kvd * 2);
                memcpy(wv + t * kvd, vc + row * kvd, kvd * 2);
            }
            orc_attention_f16(q, wk, wv, att, win - 1, (size_t)m->n_heads, (size_t)m->n_kv_heads, hd,
                              m->attn_scale);
            free(wk);
            free(wv);
        }
        orc_quantize_q8_0(att, xq, qd);
        orc_mat_vec_mul_q4_0_q8_0(m->wo[l], xq, tmp, dim, qd, isa, threads);
        orc_rms_norm(tmp, m->post_attn_norm[l], m->eps, xn, dim);
        for (size_t i = 0; i < dim; i++) h[i] = h[i] + xn[i];
        orc_rms_norm(h, m->ffn_norm[l], m->eps, xn, dim);
        orc_quantize_q8_0(xn, xq, dim);
        orc_mat_vec_mul_q4_0_q8_0(m->wgate[l], xq, g, ffn, dim, isa, threads);
        orc_mat_vec_mul_q4_0_q8_0(m->wup[l], xq, u, ffn, dim, isa, threads);
        orc_geglu(g, u, act, ffn);
        orc_quantize_q8_0(act, xq, ffn);
        orc_mat_vec_mul_q4_0_q8_0(m->wdown[l], xq, tmp, dim, ffn, isa, threads);
        orc_rms_norm(tmp, m->post_ffw_norm[l], m->eps, xn, dim);
        for (size_t i = 0; i < dim; i++) h[i] = h[i] + xn[i];
    }
    orc_rms_norm(h, m->output_norm, m->eps, xn, dim);
    orc_quantize_q8_0(xn, xq, dim);
    if (m->tie_q8) orc_mat_vec_mul_q8_0_q8_0(m->tok_embd, xq, lg, vocab, dim, 0, isa, threads);
    else orc_mat_vec_mul_q4_0_q8_0(m->tok_embd, xq, lg, vocab, dim, isa, threads);
    if (m->softcap)
        for (size_t i = 0; i < vocab; i++) lg[i] = 30.0f * tanhf(lg[i] / 30.0f);
    int64_t best = orc_argmax_f32(lg, vocab);

    free(h); free(xn); free(tmp); free(q); free(k); free(v); free(att);
    free(g); free(u); free(act); free(xq);
    if (!logits) free(lg);
    return best;
}
