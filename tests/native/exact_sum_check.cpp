// Checks qt_llama.cpp_amd/csrc/exact_sum.h: the events built from the
// per-term classification (runs of safe terms -> one exact addend, other
// terms kept) must sum sequentially to the bits of the plain loop
// s = 0; s = s + a_k, also with runs cut every 256 terms.  Approximate prefix sums come from a double-precision
// pass rounded to f32 (within the classification's error allowance).
//   exact_sum_check [cases] [seed]  -> prints "mismatches <m> cases <c> events_avg <e>"
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "../../qt_llama.cpp_amd/csrc/exact_sum.h"

static float plain(const std::vector<float> &a)
{
    float s = 0.0f;
    for (float v : a) s = s + v;
    return s;
}

// split > 0: a run is also cut where k is a multiple of split (the GPU sum
// cuts runs at every wave's first term); the parts stay exact.
static float by_events(const std::vector<float> &a, size_t &nev, int split)
{
    const int n = (int)a.size();
    std::vector<float> P(n);
    double acc = 0.0;
    for (int k = 0; k < n; ++k) {
        acc += a[k];
        P[k] = (float)acc;
    }
    std::vector<float> ev;
    bool in_run = false;
    long long R = 0;
    float u = 0.0f;
    for (int k = 0; k < n; ++k) {
        // the margin of the last term of k's group of four, as the GPU's
        // register path uses
        const float rho = mrml_xsum::margin(k | 3);
        const mrml_xsum::Step st = mrml_xsum::classify(a[k], k ? P[k - 1] : 0.0f, P[k], k == 0, 1.0f - rho, 1.0f + rho);
        if (!st.safe) {
            ev.push_back(a[k]);
            in_run = false;
            continue;
        }
        if (!in_run || st.u != u || (split > 0 && k % split == 0)) {  // a run never changes binade; the check keeps the emulation honest
            if (in_run && st.u != u) return -1.0f;
            ev.push_back(0.0f);
            R = 0;
            u = st.u;
            in_run = true;
        }
        R += st.inc;
        ev.back() = (float)R * u;
    }
    nev = ev.size();
    float s = 0.0f;
    for (float v : ev) s = s + v;
    return s;
}

int main(int argc, char **argv)
{
    const int cases = argc > 1 ? atoi(argv[1]) : 20000;
    const unsigned seed = argc > 2 ? (unsigned)atoi(argv[2]) : 1u;
    std::mt19937_64 rng(seed);
    std::normal_distribution<double> nd(0.0, 1.0);
    std::uniform_real_distribution<double> ud(0.0, 1.0);
    long long mism = 0, evsum = 0;
    for (int c = 0; c < cases; ++c) {
        const int kind = c % 7;
        const int n = 1 + (int)(ud(rng) * (kind == 6 ? 64 : 4096));
        std::vector<float> a(n);
        const double scale = std::pow(10.0, ud(rng) * 16.0 - 8.0);
        for (int k = 0; k < n; ++k) {
            double v;
            switch (kind) {
            case 0: { const float x = (float)(nd(rng) * scale); v = (double)(x * x); break; }  // squares of N(0, s)
            case 1: v = std::exp(-std::fabs(nd(rng)) * 8.0); break;                          // softmax terms
            case 2: v = ud(rng) < 0.2 ? 0.0 : (ud(rng) < 0.01 ? 1e6 * scale : scale * ud(rng)); break;
            case 3: v = std::ldexp((double)(rng() % 4096), -12); break;                      // many exact ties
            case 4: v = 1.0; break;                                                           // constant
            case 5: v = std::ldexp(ud(rng), -140); break;                                     // subnormal range
            default: v = std::ldexp(ud(rng), (int)(ud(rng) * 60.0) - 30); break;              // wide range
            }
            a[k] = (float)v;
        }
        size_t nev = 0, nev_split = 0;
        const float want = plain(a), got = by_events(a, nev, 0), got_split = by_events(a, nev_split, 256);
        evsum += (long long)nev;
        if (__builtin_bit_cast(uint32_t, want) != __builtin_bit_cast(uint32_t, got) ||
            __builtin_bit_cast(uint32_t, want) != __builtin_bit_cast(uint32_t, got_split)) {
            if (mism < 5) printf("case %d kind %d n %d: plain %a events %a split %a\n", c, kind, n, want, got, got_split);
            ++mism;
        }
    }
    printf("mismatches %lld cases %d events_avg %.1f\n", mism, cases, (double)evsum / cases);
    return mism != 0;
}
