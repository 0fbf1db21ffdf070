// tsx_half.hpp - IEEE binary16 <-> binary32 on the host (round to nearest even), for the host-side weight
// quantizers and the CPU expert rows.
#pragma once

#include <cstdint>
#include <cstring>

namespace tsx {

inline uint16_t f2h(float f) {  // IEEE binary16, round to nearest even
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t) sign;
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int) e;
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t) (sign | q);
    }
    uint32_t q = (ax - 0x38000000u) >> 13;
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t) (sign | q);
}
inline float h2f(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) return sign ? -0.0f : 0.0f;
        const float v = (float) m * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace tsx
