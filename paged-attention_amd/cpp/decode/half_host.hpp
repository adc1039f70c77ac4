#pragma once
// IEEE-754 binary16 <-> binary32 on the host, for the fp32 host-pointer
// interfaces (KVPool, AttentionBackend) that feed the fp16 cache. Written from
// the IEEE-754 formats: float -> half rounds to nearest even (ties to the even
// significand), overflows to infinity at |x| >= 65520, keeps NaN quiet and
// produces subnormals below 2^-14; half -> float is exact.

#include <cmath>
#include <cstdint>
#include <cstring>

namespace decode {

inline uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a    = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return static_cast<uint16_t>(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);   // 65520 and up round to infinity
    if (a < 0x38800000u) {                                                // below 2^-14: multiples of 2^-24
        const int e = static_cast<int>(a >> 23) - 127;
        if (e < -25) return static_cast<uint16_t>(sign);
        const uint32_t m     = (a & 0x7fffffu) | 0x800000u;               // value = m * 2^(e - 23)
        const int      shift = -(e + 1);                                  // 14 .. 24
        uint32_t       q     = m >> shift;
        const uint32_t rem   = m & ((1u << shift) - 1u);
        const uint32_t tie   = 1u << (shift - 1);
        if (rem > tie || (rem == tie && (q & 1u))) ++q;                   // may carry into the smallest normal
        return static_cast<uint16_t>(sign | q);
    }
    uint32_t       h   = (a >> 13) - (112u << 10);                        // rebias 127 -> 15
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;              // a carry moves into the exponent
    return static_cast<uint16_t>(sign | h);
}

inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e    = (h >> 10) & 0x1fu;
    const uint32_t m    = h & 0x3ffu;
    if (e == 0) {
        const float v = std::ldexp(static_cast<float>(m), -24);
        return sign ? -v : v;
    }
    const uint32_t x = e == 0x1f ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    float f;
    std::memcpy(&f, &x, sizeof f);
    return f;
}

}  // namespace decode
