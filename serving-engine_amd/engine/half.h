// half.h -- the 16-bit storage type of the C++ API.
//
// The reference passes fp16 tensors as CUDA's `half` (cuda_fp16.h).  Here a
// `half` is a plain IEEE-754 binary16 bit pattern: the host never computes in
// it, it only moves it, and device code reinterprets the same bytes as
// _Float16.  Conversions round to nearest, ties to even, and follow the
// binary16 definition (1 sign, 5 exponent bits with bias 15, 10 fraction
// bits; subnormals, infinities and NaN kept).
#pragma once

#include <cstdint>
#include <cstring>

namespace engine {

struct half {
    uint16_t bits;
};
static_assert(sizeof(half) == 2, "half must be 2 bytes");

inline float half_to_float(half h) {
    const uint32_t sign = (uint32_t)(h.bits & 0x8000u) << 16;
    const uint32_t exp = (h.bits >> 10) & 0x1fu;
    uint32_t frac = h.bits & 0x3ffu;
    uint32_t out;
    if (exp == 0x1f) {
        out = sign | 0x7f800000u | (frac << 13);           // inf / NaN
    } else if (exp != 0) {
        out = sign | ((exp + 112u) << 23) | (frac << 13);  // normal: rebias 15 -> 127
    } else if (frac == 0) {
        out = sign;                                        // signed zero
    } else {
        // subnormal: value = frac * 2^-24; normalise into a float
        int e = -1;
        do {
            frac <<= 1;
            ++e;
        } while ((frac & 0x400u) == 0);
        out = sign | ((uint32_t)(112 - e) << 23) | ((frac & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &out, 4);
    return f;
}

inline half float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {  // inf or NaN (NaN keeps a quiet payload bit)
        return half{(uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u))};
    }
    if (ax >= 0x477ff000u) return half{(uint16_t)(sign | 0x7c00u)};  // rounds past 65504
    const int exp = (int)(ax >> 23) - 127;
    if (exp >= -14) {
        // normal result: keep 10 fraction bits, round the 13 dropped bits
        uint32_t mant = ax & 0x7fffffu;
        uint32_t hb = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (hb & 1u))) ++hb;  // carry may bump exponent
        return half{(uint16_t)(sign | hb)};
    }
    if (exp < -25) return half{sign};  // below half the smallest subnormal
    // subnormal result: value / 2^-24, rounded to an integer
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;  // 24-bit significand
    const int shift = -exp - 1;                          // 14 .. 24 bits dropped
    uint32_t hb = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (hb & 1u))) ++hb;
    return half{(uint16_t)(sign | hb)};
}

}  // namespace engine
