// fp32 -> fp16 on the host, round to nearest even (the rounding of the
// library's own fp32 -> fp16 conversions), for the C++ consumers under
// tests/cxx.
#pragma once

#include <cstdint>
#include <cstring>

namespace host_half
{
inline uint16_t from_float(float f)
{
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int exp = int((x >> 23) & 0xffu) - 127 + 15;
    uint32_t mant = x & 0x7fffffu;
    if (((x >> 23) & 0xffu) == 0xffu)
        return uint16_t(sign | 0x7c00u | (mant ? 0x200u : 0u));
    if (exp >= 31)
        return uint16_t(sign | 0x7c00u);
    if (exp <= 0)
    {
        if (exp < -10)
            return uint16_t(sign);
        mant |= 0x800000u;
        const int shift = 14 - exp;
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u)))
            h++;
        return uint16_t(sign | h);
    }
    uint32_t h = (uint32_t(exp) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
        h++;
    return uint16_t(sign | h);
}
} // namespace host_half
