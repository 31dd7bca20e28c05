// Compares the f32 tanh/exp/sin/cos of qt_llama.cpp_amd/csrc/libm_f32.h with
// the host C library's tanhf/expf/sinf/cosf (the functions the reference
// links) on every float bit pattern u with u % stride == offset.  Prints
// mismatch counts:
//   tanhf <n> expf_fused <n> expf_plain <n> sinf_fused <n> sinf_plain <n>
//   cosf_fused <n> cosf_plain <n> checked <n>
// Build: g++ -O2 -std=c++17 -fopenmp -ffp-contract=off libm_check.cpp -lm
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "../../qt_llama.cpp_amd/csrc/libm_f32.h"

static bool same(float a, float b)
{
    if (a != a && b != b) return true;
    return __builtin_bit_cast(uint32_t, a) == __builtin_bit_cast(uint32_t, b);
}

int main(int argc, char **argv)
{
    const uint64_t stride = argc > 1 ? strtoull(argv[1], nullptr, 10) : 1;
    const uint64_t offset = argc > 2 ? strtoull(argv[2], nullptr, 10) : 0;
    unsigned long long bad_tanh = 0, bad_fused = 0, bad_plain = 0, n = 0;
    unsigned long long bad_sin[2] = {0, 0}, bad_cos[2] = {0, 0};
    long long first_tanh = -1, first_fused = -1, first_plain = -1;
#pragma omp parallel for schedule(static, 1 << 16) reduction(+ : bad_tanh, bad_fused, bad_plain, n, bad_sin[:2], \
                                                                 bad_cos[:2])
    for (long long i = (long long)offset; i < (1ll << 32); i += (long long)stride) {
        const float x = __builtin_bit_cast(float, (uint32_t)i);
        ++n;
        if (!same(::tanhf(x), mrml_libm::tanhf(x))) {
            ++bad_tanh;
            if (first_tanh < 0) first_tanh = i;
        }
        const float e = ::expf(x);
        if (!same(e, mrml_libm::expf(x, true))) {
            ++bad_fused;
            if (first_fused < 0) first_fused = i;
        }
        if (!same(e, mrml_libm::expf(x, false))) {
            ++bad_plain;
            if (first_plain < 0) first_plain = i;
        }
        const float s = ::sinf(x), c = ::cosf(x);
        for (int f = 0; f < 2; ++f) {
            bad_sin[f] += !same(s, mrml_libm::sinf(x, f == 0));
            bad_cos[f] += !same(c, mrml_libm::cosf(x, f == 0));
        }
    }
    printf("tanhf %llu expf_fused %llu expf_plain %llu sinf_fused %llu sinf_plain %llu cosf_fused %llu cosf_plain %llu "
           "checked %llu\n",
           bad_tanh, bad_fused, bad_plain, bad_sin[0], bad_sin[1], bad_cos[0], bad_cos[1], n);
    if (first_tanh >= 0) printf("first tanhf mismatch 0x%08llx\n", (unsigned long long)first_tanh);
    if (first_fused >= 0) printf("first expf_fused mismatch 0x%08llx\n", (unsigned long long)first_fused);
    if (first_plain >= 0) printf("first expf_plain mismatch 0x%08llx\n", (unsigned long long)first_plain);
    return 0;
}
