// libm_check.cpp -- hero/libm.hpp on the host against glibc's expf / log1pf.
// Usage: libm_check STRIDE   (1 = all 2^32 bit patterns, about a minute)
// Prints "<count> <exp mismatches> <log1p mismatches>" and exits 0 iff both are 0.
#include <cstdio>
#include <cstdlib>
#include <initializer_list>

#include "hero/libm.hpp"

int main(int argc, char** argv) {
    const uint64_t stride = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
    long n = 0, be = 0, bl = 0;
    auto one = [&](uint32_t u) {
        const float x = hero::bits_f32(u);
        if (std::isnan(x)) return;
        ++n;
        if (hero::f32_bits(std::exp(x)) != hero::f32_bits(hero::expf_glibc(x))) ++be;
        const float g = std::log1p(x), m = hero::log1pf_glibc(x);
        if (hero::f32_bits(g) != hero::f32_bits(m) && !(std::isnan(g) && std::isnan(m))) ++bl;
    };
    for (uint64_t b = 0; b < (1ull << 32); b += stride) one(uint32_t(b));
    // inputs where a last-bit difference from the correctly rounded value is known
    for (uint32_t u : std::initializer_list<uint32_t>{0x4202422fu, 0xc27c65d9u, 0x3ed413d7u, 0x3ed413dau, 0x7e3504f3u, 0x42b17218u, 0xc2cff1b5u}) one(u);
    std::printf("%ld %ld %ld\n", n, be, bl);
    return (be == 0 && bl == 0) ? 0 : 1;
}
