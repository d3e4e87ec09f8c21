// seqsum_check.cpp -- the workgroup sum of hero/seqsum.hpp, run phase by phase
// on the host (1024-, 512- and 256-lane forms), against the plain sequential loop,
// bit for bit.
// Usage: seqsum_check TRIALS   prints "<trials> <mismatches> <fallbacks>"
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "hero/seqsum.hpp"

using namespace hero;

int main(int argc, char** argv) {
    const int trials = argc > 1 ? std::atoi(argv[1]) : 1000;
    std::mt19937_64 rng(12345);
    std::normal_distribution<float> N01(0.f, 1.f);
    std::uniform_real_distribution<float> U01(0.f, 1.f);
    static seqsum::Shared sm;
    long bad = 0, fallbacks = 0, fb_kind[11] = {0};
    std::vector<float> p(seqsum::kMaxN);
    for (int t = 0; t < trials; ++t) {
        const int kind = t % 11;
        int n = kind < 5 ? seqsum::kMaxN : 1 + int(rng() % seqsum::kMaxN);
        if (t % 97 == 0) n = 1 + int(rng() % 40);
        const float scale = std::ldexp(1.f, int(rng() % 60) - 30);
        for (int i = 0; i < n; ++i) {
            float x = N01(rng) * scale;
            switch (kind) {
                case 0: case 1: case 5: p[i] = x * x; break;                           // sums of squares
                case 2: p[i] = 1.f; break;                                             // exact until 2^24
                case 3: p[i] = float(int(U01(rng) * 8)) * 0.5f * scale; break;         // many ties
                case 4: p[i] = (i % 7 == 0) ? 0.f : x * x; break;                      // zeros
                case 6: p[i] = U01(rng) < 0.01f ? x * x * 1e6f : x * x; break;          // outliers
                case 7: p[i] = std::ldexp(1.f, int(rng() % 40) - 20) * (1.f + float(rng() % 4) / 4); break;
                case 8: p[i] = x * x * 1e-30f; break;                                  // subnormal range
                case 9: p[i] = (i < 8) ? 0.f : std::fabs(x); break;                    // leading zeros
                default: p[i] = i == 0 ? 3000.f * U01(rng) : std::exp(-4.f * std::fabs(N01(rng))); break;  // softmax chunk
            }
        }
        if (t % 211 == 0) p[rng() % n] = INFINITY;
        if (t % 307 == 0) p[rng() % n] = NAN;
        const float want = seqsum::serial_loop(p.data(), n);
        // rotate through the 1024-, 512- and 256-lane workgroup forms
        const float got = t % 3 == 1 ? seqsum::sum_nonneg_host<256>(p.data(), n, sm)
                          : t % 3 == 2 ? seqsum::sum_nonneg_host<512>(p.data(), n, sm)
                                       : seqsum::sum_nonneg_host<1024>(p.data(), n, sm);
        uint32_t a, b;
        std::memcpy(&a, &want, 4);
        std::memcpy(&b, &got, 4);
        if (a != b && !(want != want && got != got)) {
            if (bad < 5) std::printf("mismatch trial %d kind %d n %d: want %a got %a\n", t, kind, n, want, got);
            ++bad;
        }
        fallbacks += sm.fell_back;
        fb_kind[kind] += sm.fell_back;
    }
    std::printf("%d %ld %ld\n", trials, bad, fallbacks);
    if (argc > 2)
        for (int k = 0; k < 11; ++k) std::fprintf(stderr, "kind %d fallbacks %ld\n", k, fb_kind[k]);
    return bad == 0 ? 0 : 1;
}
