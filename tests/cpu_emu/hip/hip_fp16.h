// CPU emulation of the half-precision helpers the kernels use (test only).
#pragma once
#include <cstdint>
#include <cstring>

struct __half {
    uint16_t bits;
};
inline __half __float2half_rn(float v) {
    _Float16 h = (_Float16)v;  // round to nearest even
    __half out;
    std::memcpy(&out.bits, &h, 2);
    return out;
}
inline uint16_t __half_as_ushort(__half h) { return h.bits; }
inline __half __ushort_as_half(uint16_t bits) {
    __half out;
    out.bits = bits;
    return out;
}
inline float __half2float(__half h) {
    _Float16 v;
    std::memcpy(&v, &h.bits, 2);
    return (float)v;
}
