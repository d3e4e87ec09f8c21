// fp16.hpp -- the half-precision codec the Q8_0 path depends on, for host and
// device.
//
// Decode is plain IEEE binary16 -> binary32 and is exact; on the device the
// hardware conversion is used. Encode restates nm/src/core.hpp:61-79: it
// rounds half-up in magnitude on the first dropped bit (no sticky bits, so it
// is NOT round-to-nearest-even) and maps NaN to Inf. The Q8_0 activation scale
// is stored through this encoder, so the device must use the same integer
// steps rather than a hardware conversion.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace hero {

__host__ __device__ inline uint32_t f32_bits(float f) {
    union {
        float f;
        uint32_t u;
    } v{f};
    return v.u;
}
__host__ __device__ inline float bits_f32(uint32_t u) {
    union {
        uint32_t u;
        float f;
    } v{u};
    return v.f;
}

__host__ __device__ inline uint16_t fp32_to_fp16_ref(float f) {
    const uint32_t x = f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t exponent = int32_t((x >> 23) & 0xFFu) - 112;
    uint32_t mantissa = x & 0x7FFFFFu;
    if (exponent <= 0) {
        if (exponent < -10) return uint16_t(sign);
        mantissa |= 0x800000u;
        const uint32_t shift = uint32_t(14 - exponent);
        const uint32_t r = (mantissa >> shift) + ((mantissa >> (shift - 1)) & 1u);
        return uint16_t(sign | r);
    }
    if (exponent >= 0x1F) return uint16_t(sign | 0x7C00u);
    const uint32_t h = sign | (uint32_t(exponent) << 10) | (mantissa >> 13);
    return uint16_t(h + ((mantissa >> 12) & 1u));
}

// Exact IEEE decode (integer form, used on the host).
__host__ __device__ inline float fp16_to_fp32_ref(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1Fu) return bits_f32(sign | 0x7F800000u | (m << 13));
    if (e != 0) return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
    // zero or subnormal: m * 2^-24, exact in fp32
    const float mag = float(m) * 5.9604644775390625e-08f;
    return sign ? -mag : mag;
}

}  // namespace hero
