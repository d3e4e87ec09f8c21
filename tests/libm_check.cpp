// libm_check.cpp -- hero/libm.hpp on the host against glibc's expf / log1pf /
// expm1f / tanhf.
// Usage: libm_check STRIDE   (1 = all 2^32 bit patterns, a few minutes)
// Prints "<count> <exp> <log1p> <expm1> <tanh>" (mismatch counts) and exits 0
// iff all four are 0.
#include <cstdio>
#include <cstdlib>
#include <initializer_list>

#include "hero/libm.hpp"

int main(int argc, char** argv) {
    const uint64_t stride = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
    long n = 0, be = 0, bl = 0, bm = 0, bt = 0;
    auto one = [&](uint32_t u) {
        const float x = hero::bits_f32(u);
        if (std::isnan(x)) return;
        ++n;
        if (hero::f32_bits(std::exp(x)) != hero::f32_bits(hero::expf_glibc(x))) ++be;
        const float g = std::log1p(x), m = hero::log1pf_glibc(x);
        if (hero::f32_bits(g) != hero::f32_bits(m) && !(std::isnan(g) && std::isnan(m))) ++bl;
        if (hero::f32_bits(std::expm1(x)) != hero::f32_bits(hero::expm1f_glibc(x))) ++bm;
        if (hero::f32_bits(std::tanh(x)) != hero::f32_bits(hero::tanhf_glibc(x))) ++bt;
    };
    for (uint64_t b = 0; b < (1ull << 32); b += stride) one(uint32_t(b));
    // inputs where a last-bit difference from the correctly rounded value is known
    for (uint32_t u : std::initializer_list<uint32_t>{0x4202422fu, 0xc27c65d9u, 0x3ed413d7u, 0x3ed413dau, 0x7e3504f3u, 0x42b17218u, 0xc2cff1b5u,
                                                 // expm1f / tanhf branch edges: 27 ln2, 88.72, ln2/2, 1.5 ln2, 2^-25, 1, 22, 2^-55
                                                 0x4195b844u, 0xc195b844u, 0x42b17180u, 0x42b17181u, 0x3eb17218u, 0x3eb17219u, 0x3f851592u,
                                                 0xbf851592u, 0x33000000u, 0x3f800000u, 0xbf800000u, 0x41b00000u, 0xc1b00000u, 0x24000000u}) one(u);
    std::printf("%ld %ld %ld %ld %ld\n", n, be, bl, bm, bt);
    return (be == 0 && bl == 0 && bm == 0 && bt == 0) ? 0 : 1;
}
